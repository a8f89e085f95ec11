// barracuda_hip_ops.hpp -- C++17 host API over libbarracuda_hip (barracuda_hip.h).
//
// Mirrors the reference's Rust op surface for the dense ML-ops hot path
// (ecoPrimals/barraCuda, paths relative to crates/barracuda/src/): the same
// method names, argument meaning, validation order and error variants, so
// that code and tests written against the reference read the same here.
//
//   Tensor::{from_data, from_vec_on, shape, len, to_vec}   tensor/mod.rs:185, 347, 409, 448
//   Tensor::matmul / matmul_ref, MatMul                    ops/matmul.rs:49-243
//   Tensor::matmul_tiled, MatmulTiled                      ops/matmul_tiled.rs:45-171
//   Tensor::batch_matmul, BatchMatMul                      ops/batch_matmul.rs:24-163
//   Tensor::softmax, Softmax (global)                      ops/softmax.rs:31-144
//   Tensor::softmax_dim                                    ops/tensor_axis_ops.rs:67-126
//   Tensor::attention, Attention                           ops/attention/mod.rs:84-206
//   Tensor::scaled_dot_product_attention                   ops/scaled_dot_product_attention/mod.rs:81-226
//   Tensor::causal_attention, CausalAttention              ops/causal_attn/mod.rs:64-158
//   FlashAttention                                         ops/flash_attention.rs:45-146
//   Tensor::grouped_query_attention, GroupedQueryAttention ops/grouped_query_attention/mod.rs:52-226
//   Tensor::multi_head_attention, MultiHeadAttention       ops/mha/mod.rs:48-263, projections.rs:18-58
//   Tensor::reshape                                        tensor/mod.rs (shape-only view)
//   nn::fused_mlp, nn::Activation                          nn/fused_mlp.rs:25-168
//   GemmF64, GemmCachedF64                                 ops/linalg/gemm_f64.rs:77-456
//   TensorSession, SessionTensor, AttentionDims            session/mod.rs:60-540, session/tensor.rs:14-68
//   BarracudaError, Result<T>                              error.rs:14-130
//
// Every computation goes through the C ABI to the gfx950 kernels; there is
// no host fallback.  Shape validation happens here, before any device call,
// exactly where the reference does it.  Errors are values (Result<T>), as in
// Rust; unwrap() on an error throws std::runtime_error with the message.
#pragma once

#include <algorithm>
#include <array>
#include <climits>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <memory>
#include <mutex>
#include <optional>
#include <sstream>
#include <stdexcept>
#include <string>
#include <utility>
#include <variant>
#include <vector>

#include "barracuda_hip.h"

namespace barracuda {

// ---------------------------------------------------------------- errors
enum class ErrorKind {
  Device,                // error.rs Device(String)
  ShapeMismatch,         // ShapeMismatch{expected, actual}
  InvalidOperation,      // InvalidOperation{op, reason}
  InvalidInput,          // InvalidInput{message}
  OutOfMemory,           // OutOfMemory(String)
  ExecutionError,        // ExecutionError{message}
  UnsupportedOperation,  // UnsupportedOperation{op, device}
  DeviceLost,            // DeviceLost(String)
  DeviceNotAvailable,    // DeviceNotAvailable{device, reason}
  InvalidShape,          // InvalidShape{expected, actual}
  CastOverflow,          // CastOverflow{from_type, to_type, value_description}
};

inline std::string shape_str(const std::vector<size_t>& s) {
  std::ostringstream o;
  o << '[';
  for (size_t i = 0; i < s.size(); ++i) o << (i ? ", " : "") << s[i];
  o << ']';
  return o.str();
}

struct BarracudaError {
  ErrorKind kind;
  std::string message;  // rendered as the reference's #[error(...)] strings

  static BarracudaError shape_mismatch(const std::vector<size_t>& expected, const std::vector<size_t>& actual) {
    return {ErrorKind::ShapeMismatch,
            "Shape mismatch: expected " + shape_str(expected) + ", got " + shape_str(actual)};
  }
  static BarracudaError invalid_shape(const std::vector<size_t>& expected, const std::vector<size_t>& actual) {
    return {ErrorKind::InvalidShape, "Invalid shape: expected " + shape_str(expected) + ", got " + shape_str(actual)};
  }
  static BarracudaError cast_overflow(const std::string& from, const std::string& to, const std::string& value) {
    return {ErrorKind::CastOverflow, "Cast overflow: " + from + " → " + to + " (" + value + ")"};
  }
  static BarracudaError invalid_op(const std::string& op, const std::string& reason) {
    return {ErrorKind::InvalidOperation, "Invalid operation: " + op + " - " + reason};
  }
  static BarracudaError invalid_input(const std::string& msg) {
    return {ErrorKind::InvalidInput, "Invalid input: " + msg};
  }
  static BarracudaError device(const std::string& msg) { return {ErrorKind::Device, "Device error: " + msg}; }
  static BarracudaError unsupported(const std::string& op, const std::string& dev) {
    return {ErrorKind::UnsupportedOperation, "Operation not supported on device: " + op + " on " + dev};
  }
  static BarracudaError device_lost(const std::string& msg) {
    return {ErrorKind::DeviceLost, "GPU device lost: " + msg};
  }
  static BarracudaError device_not_available(const std::string& dev, const std::string& reason) {
    return {ErrorKind::DeviceNotAvailable, "Device not available: " + dev + " - " + reason};
  }
  // bch_status -> BarracudaError variant (error.rs:14-130)
  static BarracudaError from_status(bch_status st, const std::string& detail, const std::string& op) {
    switch (st) {
      case BCH_E_INVALID: return invalid_input(detail);
      case BCH_E_SHAPE: return invalid_op(op, "shape/dimension mismatch: " + detail);
      case BCH_E_NO_DEVICE: return device_not_available("hip", detail);
      case BCH_E_OOM: return {ErrorKind::OutOfMemory, "Out of memory: " + detail};
      case BCH_E_LAUNCH: return {ErrorKind::ExecutionError, "Execution error: " + detail};
      case BCH_E_UNSUPPORTED: return unsupported(op, "hip:gfx950 (" + detail + ")");
      case BCH_E_DEVICE_LOST: return device_lost(detail);
      default: return device(detail);  // BCH_E_MODULE, BCH_E_DEVICE
    }
  }
};

template <class T>
class Result {
 public:
  Result(T v) : v_(std::move(v)) {}                   // NOLINT: implicit like Ok(..)
  Result(BarracudaError e) : v_(std::move(e)) {}      // NOLINT: implicit like Err(..)
  bool is_ok() const { return v_.index() == 0; }
  bool is_err() const { return v_.index() == 1; }
  const BarracudaError& error() const { return std::get<1>(v_); }
  T& value() { return std::get<0>(v_); }
  T unwrap() && {
    if (is_err()) throw std::runtime_error(error().message);
    return std::move(std::get<0>(v_));
  }
  T unwrap() & {
    if (is_err()) throw std::runtime_error(error().message);
    return std::get<0>(v_);
  }

 private:
  std::variant<T, BarracudaError> v_;
};

// ---------------------------------------------------------------- device
// One bch_ctx (device + stream): the device half of GpuBackend
// (device/backend.rs:244-444).  Calls are serialised: a context is not
// re-entrant.
class HipDevice {
 public:
  static Result<std::shared_ptr<HipDevice>> create(int ordinal = -1) {
    bch_ctx* ctx = nullptr;
    const bch_status st = bch_ctx_create(ordinal, nullptr, &ctx);
    if (st != BCH_OK) return BarracudaError::from_status(st, bch_last_error(nullptr), "device");
    return std::shared_ptr<HipDevice>(new HipDevice(ctx));
  }
  ~HipDevice() { bch_ctx_destroy(ctx_); }
  HipDevice(const HipDevice&) = delete;
  HipDevice& operator=(const HipDevice&) = delete;

  std::string name() const { return "hip:gfx950"; }
  // GpuBackend::is_lost (device/backend.rs:256)
  bool is_lost() const {
    int lost = 0;
    return bch_ctx_is_lost(ctx_, &lost) == BCH_OK && lost != 0;
  }
  bch_ctx* ctx() const { return ctx_; }
  std::mutex& mutex() { return mu_; }
  std::optional<BarracudaError> check(bch_status st, const std::string& op) const {
    if (st == BCH_OK) return std::nullopt;
    return BarracudaError::from_status(st, bch_last_error(ctx_), op);
  }

 private:
  explicit HipDevice(bch_ctx* c) : ctx_(c) {}
  bch_ctx* ctx_;
  std::mutex mu_;
};

namespace detail {
// Owned device allocation (RAII bch_free), shared between Tensor clones.
struct DeviceBuffer {
  std::shared_ptr<HipDevice> dev;
  void* ptr = nullptr;
  size_t bytes = 0;
  ~DeviceBuffer() {
    if (ptr) {
      std::lock_guard<std::mutex> g(dev->mutex());
      bch_free(dev->ctx(), ptr);
    }
  }
};

inline size_t numel(const std::vector<size_t>& s) {
  size_t n = 1;
  for (size_t d : s) n *= d;
  return n;
}

// The C ABI takes GEMM / attention dimensions as int.
inline std::optional<BarracudaError> check_i32(const char* op, std::initializer_list<size_t> dims) {
  for (size_t d : dims)
    if (d > (size_t)INT_MAX)
      return BarracudaError::unsupported(op, "hip:gfx950 (dimension " + std::to_string(d) + " exceeds 2^31-1)");
  return std::nullopt;
}
}  // namespace detail

// ---------------------------------------------------------------- tensor
class Tensor {
 public:
  // tensor/mod.rs:185 from_data: upload f32 data with a shape
  static Result<Tensor> from_data(const std::vector<float>& data, std::vector<size_t> shape,
                                  const std::shared_ptr<HipDevice>& dev) {
    if (data.size() != detail::numel(shape))
      return BarracudaError::shape_mismatch({detail::numel(shape)}, {data.size()});
    auto r = empty(std::move(shape), dev);
    if (r.is_err()) return r;
    Tensor t = std::move(r).unwrap();
    if (!data.empty()) {
      std::lock_guard<std::mutex> g(dev->mutex());
      if (auto e = dev->check(bch_upload(dev->ctx(), t.buf_->ptr, data.data(), data.size() * sizeof(float)),
                              "upload"))
        return *e;
    }
    return t;
  }
  static Result<Tensor> from_vec_on(const std::vector<float>& data, std::vector<size_t> shape,
                                    const std::shared_ptr<HipDevice>& dev) {
    return from_data(data, std::move(shape), dev);
  }
  // an uninitialised output tensor (the reference's pooled output buffers)
  static Result<Tensor> empty(std::vector<size_t> shape, const std::shared_ptr<HipDevice>& dev) {
    auto buf = std::make_shared<detail::DeviceBuffer>();
    buf->dev = dev;
    buf->bytes = detail::numel(shape) * sizeof(float);
    if (buf->bytes) {
      std::lock_guard<std::mutex> g(dev->mutex());
      if (auto e = dev->check(bch_alloc(dev->ctx(), buf->bytes, &buf->ptr), "alloc_buffer")) return *e;
    }
    return Tensor(std::move(buf), std::move(shape), dev);
  }

  const std::vector<size_t>& shape() const { return shape_; }
  size_t len() const { return detail::numel(shape_); }
  const std::shared_ptr<HipDevice>& device() const { return dev_; }
  float* data_ptr() const { return static_cast<float*>(buf_->ptr); }

  // tensor/mod.rs:448 to_vec: blocking readback
  Result<std::vector<float>> to_vec() const {
    std::vector<float> out(len());
    if (!out.empty()) {
      std::lock_guard<std::mutex> g(dev_->mutex());
      if (auto e = dev_->check(bch_download(dev_->ctx(), out.data(), buf_->ptr, out.size() * sizeof(float)),
                               "download"))
        return *e;
    }
    return out;
  }

  inline Result<Tensor> matmul(const Tensor& other) const;
  inline Result<Tensor> matmul_ref(const Tensor& other) const;
  inline Result<Tensor> matmul_tiled(const Tensor& other) const;
  inline Result<Tensor> batch_matmul(const Tensor& other) const;
  inline Result<Tensor> softmax() const;
  inline Result<Tensor> softmax_dim(size_t axis) const;
  inline Result<Tensor> relu() const;                           // ops/relu.rs:106
  inline Result<Tensor> gelu_wgsl() const;                      // ops/gelu_wgsl.rs:147
  inline Result<Tensor> layer_norm_wgsl(float epsilon) const;   // ops/layer_norm_wgsl.rs:160-165
  inline Result<Tensor> attention(const Tensor& key, const Tensor& value) const;
  inline Result<Tensor> scaled_dot_product_attention(const Tensor& key, const Tensor& value) const;
  inline Result<Tensor> causal_attention(const Tensor& key, const Tensor& value) const;
  inline Result<Tensor> grouped_query_attention(const Tensor& key, const Tensor& value) const;
  inline Result<Tensor> multi_head_attention(const Tensor& key, const Tensor& value, const Tensor& w_q,
                                             const Tensor& w_k, const Tensor& w_v, const Tensor& w_o,
                                             size_t num_heads) const;

  // A tensor with a shape and no buffer or device: for validation-only
  // tests of the op structs (nothing may read its data).
  static Tensor null_for_tests(std::vector<size_t> shape) { return Tensor(nullptr, std::move(shape), nullptr); }

  // Same buffer under a new shape with the same element count (used by
  // MultiHeadAttention, ops/mha/projections.rs:32-35).
  Result<Tensor> reshape(std::vector<size_t> shape) const {
    if (detail::numel(shape) != len()) return BarracudaError::shape_mismatch(shape, shape_);
    return Tensor(buf_, std::move(shape), dev_);
  }

 private:
  Tensor(std::shared_ptr<detail::DeviceBuffer> b, std::vector<size_t> s, std::shared_ptr<HipDevice> d)
      : buf_(std::move(b)), shape_(std::move(s)), dev_(std::move(d)) {}
  std::shared_ptr<detail::DeviceBuffer> buf_;
  std::vector<size_t> shape_;
  std::shared_ptr<HipDevice> dev_;
};

// ---------------------------------------------------------------- ops
// ops/matmul.rs:92-114: 2D+ inputs (>= 3-D use shape[0..2]), inner dims equal.
struct MatMul {
  const Tensor& lhs;
  const Tensor& rhs;
  static std::optional<BarracudaError> validate(const std::vector<size_t>& ls, const std::vector<size_t>& rs) {
    if (ls.size() < 2 || rs.size() < 2)
      return BarracudaError::invalid_op("matmul", "requires 2D+ tensors, got shapes " + shape_str(ls) + " and " +
                                                      shape_str(rs));
    if (ls[1] != rs[0]) return BarracudaError::shape_mismatch(ls, rs);
    return std::nullopt;
  }
  Result<Tensor> execute() const {
    if (auto e = validate(lhs.shape(), rhs.shape())) return *e;
    if (auto e = detail::check_i32("matmul", {lhs.shape()[0], lhs.shape()[1], rhs.shape()[1]})) return *e;
    const int m = (int)lhs.shape()[0], k = (int)lhs.shape()[1], n = (int)rhs.shape()[1];
    auto dev = lhs.device();
    auto r = Tensor::empty({(size_t)m, (size_t)n}, dev);
    if (r.is_err() || m == 0 || n == 0) return r;
    Tensor out = std::move(r).unwrap();
    std::lock_guard<std::mutex> g(dev->mutex());
    const int lk = k > 1 ? k : 1, ln = n > 1 ? n : 1;
    if (auto e = dev->check(bch_sgemm(dev->ctx(), m, n, k, lhs.data_ptr(), lk, rhs.data_ptr(), ln, out.data_ptr(), ln),
                            "matmul"))
      return *e;
    return out;
  }
};
using MatmulTiled = MatMul;  // ops/matmul_tiled.rs: same contract

// ops/batch_matmul.rs:47-144: A[batch,m,k] . B[batch,k,n].  The reference
// does not check B against A; a disagreeing B is a ShapeMismatch here.
struct BatchMatMul {
  const Tensor& a;
  const Tensor& b;
  static std::optional<BarracudaError> validate(const std::vector<size_t>& as, const std::vector<size_t>& bs) {
    if (as.size() != 3 || bs.size() != 3)
      return BarracudaError::invalid_op("batch_matmul", "requires 3D tensors, got shapes " + shape_str(as) +
                                                            " and " + shape_str(bs));
    if (bs[0] != as[0] || bs[1] != as[2]) return BarracudaError::shape_mismatch(as, bs);
    return std::nullopt;
  }
  Result<Tensor> execute() const {
    if (auto e = validate(a.shape(), b.shape())) return *e;
    if (auto e = detail::check_i32("batch_matmul", {a.shape()[0], a.shape()[1], a.shape()[2], b.shape()[2]})) return *e;
    const int batch = (int)a.shape()[0], m = (int)a.shape()[1], k = (int)a.shape()[2], n = (int)b.shape()[2];
    auto dev = a.device();
    auto r = Tensor::empty({(size_t)batch, (size_t)m, (size_t)n}, dev);
    if (r.is_err() || (size_t)batch * m * n == 0) return r;
    Tensor out = std::move(r).unwrap();
    std::lock_guard<std::mutex> g(dev->mutex());
    if (auto e = dev->check(bch_sgemm_strided_batched(dev->ctx(), batch, m, n, k, a.data_ptr(), (long long)m * k,
                                                      b.data_ptr(), (long long)k * n, out.data_ptr(),
                                                      (long long)m * n),
                            "batch_matmul"))
      return *e;
    return out;
  }
};

// ops/softmax.rs:39-48 (non-empty shape), :58-133 (one softmax over all elements)
struct Softmax {
  const Tensor& input;
  static std::optional<BarracudaError> validate(const std::vector<size_t>& s) {
    if (s.empty()) return BarracudaError::invalid_op("Softmax", "Empty tensor not supported");
    return std::nullopt;
  }
  Result<Tensor> execute() const {
    if (auto e = validate(input.shape())) return *e;
    auto dev = input.device();
    auto r = Tensor::empty(input.shape(), dev);
    if (r.is_err() || input.len() == 0) return r;
    Tensor out = std::move(r).unwrap();
    std::lock_guard<std::mutex> g(dev->mutex());
    if (auto e = dev->check(bch_softmax_rows(dev->ctx(), 1, (long long)input.len(), input.data_ptr(), out.data_ptr()),
                            "softmax"))
      return *e;
    return out;
  }
};

// ops/tensor_axis_ops.rs:67-82: validation of softmax_dim
inline std::optional<BarracudaError> validate_softmax_dim(const std::vector<size_t>& s, size_t axis) {
  if (s.empty()) return BarracudaError::invalid_op("softmax_dim", "Empty tensor not supported");
  if (axis >= s.size())
    return BarracudaError::invalid_op("softmax_dim",
                                      "Axis " + std::to_string(axis) + " out of bounds for shape " + shape_str(s));
  return std::nullopt;
}

namespace detail {
// one element-wise op (bch_elementwise) from `in` into a new tensor of its shape
inline Result<Tensor> unary(const Tensor& in, int op, const char* name) {
  auto dev = in.device();
  auto r = Tensor::empty(in.shape(), dev);
  if (r.is_err() || in.len() == 0) return r;
  Tensor out = std::move(r).unwrap();
  std::lock_guard<std::mutex> g(dev->mutex());
  if (auto e = dev->check(bch_elementwise(dev->ctx(), op, (long long)in.len(), in.data_ptr(), nullptr, nullptr, 0.0f,
                                          out.data_ptr()),
                          name))
    return *e;
  return out;
}
}  // namespace detail

// ops/relu.rs: max(x, 0) over every element (relu_f64.wgsl)
struct ReLU {
  const Tensor& input;
  Result<Tensor> execute() const { return detail::unary(input, BCH_EW_RELU, "relu"); }
};

// ops/gelu_wgsl.rs:33-141: 0.5 x (1 + tanh(0.7978845608 (x + 0.044715 x^3)))
// over every element (gelu_f64.wgsl)
struct GELU {
  const Tensor& input;
  Result<Tensor> execute() const { return detail::unary(input, BCH_EW_GELU, "gelu"); }
};

// ops/layer_norm_wgsl.rs:47-157: each row along the last dimension becomes
// (x - mean) / sqrt(var + epsilon), biased variance, no affine parameters
// (layer_norm_f64.wgsl)
struct LayerNorm {
  const Tensor& input;
  float epsilon;
  static std::optional<BarracudaError> validate(const std::vector<size_t>& s) {
    if (s.empty()) return BarracudaError::invalid_op("LayerNorm", "Empty tensor not supported");
    return std::nullopt;
  }
  Result<Tensor> execute() const {
    if (auto e = validate(input.shape())) return *e;
    auto dev = input.device();
    auto r = Tensor::empty(input.shape(), dev);
    if (r.is_err() || input.len() == 0) return r;
    Tensor out = std::move(r).unwrap();
    const size_t cols = input.shape().back(), rows = input.len() / cols;
    std::lock_guard<std::mutex> g(dev->mutex());
    if (auto e = dev->check(bch_layer_norm(dev->ctx(), (long long)rows, (long long)cols, epsilon, input.data_ptr(),
                                           out.data_ptr()),
                            "layer_norm"))
      return *e;
    return out;
  }
};

namespace detail {
inline Result<Tensor> sdpa(const Tensor& q, const Tensor& k, const Tensor& v, bool causal, const char* op, size_t B,
                           size_t H, size_t Sq, size_t Skv, size_t D) {
  auto dev = q.device();
  if (auto e = check_i32(op, {B, H, Sq, Skv, D})) return *e;
  auto r = Tensor::empty(q.shape(), dev);
  if (r.is_err() || (size_t)B * H * Sq * D == 0) return r;
  if (Skv == 0) return BarracudaError::invalid_op(op, "key sequence is empty (shape/dimension mismatch)");
  Tensor out = std::move(r).unwrap();
  const float scale = 1.0f / std::sqrt((float)D);
  std::lock_guard<std::mutex> g(dev->mutex());
  if (auto e = dev->check(bch_sdpa_fwd(dev->ctx(), (int)B, (int)H, (int)Sq, (int)Skv, (int)D, scale, causal ? 1 : 0,
                                       q.data_ptr(), k.data_ptr(),
                                       v.data_ptr(), out.data_ptr()),
                          op))
    return *e;
  return out;
}
}  // namespace detail

// ops/attention/mod.rs:96-144: 4-D Q, K, V; batch, heads and head_dim of Q and
// K equal (Sq may differ from Skv); K and V identical shapes.
struct Attention {
  const Tensor& q;
  const Tensor& k;
  const Tensor& v;
  static std::optional<BarracudaError> validate(const std::vector<size_t>& qs, const std::vector<size_t>& ks,
                                                const std::vector<size_t>& vs) {
    const char* names[3] = {"query", "key", "value"};
    const std::vector<size_t>* ss[3] = {&qs, &ks, &vs};
    for (int i = 0; i < 3; ++i)
      if (ss[i]->size() != 4)
        return BarracudaError::invalid_op("attention", std::string(names[i]) +
                                                           " requires 4D tensor [batch, heads, seq_len, head_dim], got " +
                                                           std::to_string(ss[i]->size()) + "D");
    if (qs[0] != ks[0] || qs[1] != ks[1] || qs[3] != ks[3]) return BarracudaError::shape_mismatch(qs, ks);
    if (ks != vs) return BarracudaError::shape_mismatch(ks, vs);
    return std::nullopt;
  }
  Result<Tensor> execute() const {
    if (auto e = validate(q.shape(), k.shape(), v.shape())) return *e;
    const auto& s = q.shape();
    return detail::sdpa(q, k, v, false, "attention", s[0], s[1], s[2], k.shape()[2], s[3]);
  }
};

// ops/scaled_dot_product_attention/mod.rs:101-149: self-attention, equal shapes
struct ScaledDotProductAttention {
  const Tensor& q;
  const Tensor& k;
  const Tensor& v;
  static std::optional<BarracudaError> validate(const std::vector<size_t>& qs, const std::vector<size_t>& ks,
                                                const std::vector<size_t>& vs) {
    if (qs.size() != 4 || ks.size() != 4 || vs.size() != 4)
      return BarracudaError::invalid_input("Q, K, V must be 4D tensors [batch, heads, seq_len, head_dim]");
    if (ks != qs || vs != qs) return BarracudaError::shape_mismatch(qs, ks == qs ? vs : ks);
    return std::nullopt;
  }
  Result<Tensor> execute() const {
    if (auto e = validate(q.shape(), k.shape(), v.shape())) return *e;
    if (q.device() != k.device() || q.device() != v.device())
      return BarracudaError::device("Q, K, V must be on the same device");
    const auto& s = q.shape();
    return detail::sdpa(q, k, v, false, "scaled_dot_product_attention", s[0], s[1], s[2], s[2], s[3]);
  }
};

// ops/causal_attn/mod.rs:78-95.  The reference's GPU dispatch computes only
// rows < 16 of head 0; this follows its CPU definition
// (ops/causal_attention.rs:52-134) for every row and head.
struct CausalAttention {
  const Tensor& q;
  const Tensor& k;
  const Tensor& v;
  static std::optional<BarracudaError> validate(const std::vector<size_t>& qs, const std::vector<size_t>& ks,
                                                const std::vector<size_t>& vs) {
    if (qs.size() != 4 || ks.size() != 4 || vs.size() != 4) return BarracudaError::shape_mismatch(qs, ks);
    if (qs != ks || qs != vs) return BarracudaError::shape_mismatch(qs, ks);
    return std::nullopt;
  }
  Result<Tensor> execute() const {
    if (auto e = validate(q.shape(), k.shape(), v.shape())) return *e;
    const auto& s = q.shape();
    return detail::sdpa(q, k, v, true, "causal_attention", s[0], s[1], s[2], s[2], s[3]);
  }
};

// ops/flash_attention.rs:57-80: 2-D [seq_len, head_dim], one head, scale
// 1/sqrt(head_dim).  The reference shader keeps at most 256 keys; every key
// is attended to here (the two agree for seq_len <= 256).
struct FlashAttention {
  const Tensor& q;
  const Tensor& k;
  const Tensor& v;
  unsigned num_heads = 1;
  static std::optional<BarracudaError> validate(const std::vector<size_t>& qs, const std::vector<size_t>& ks,
                                                const std::vector<size_t>& vs) {
    if (qs != ks || qs != vs)
      return BarracudaError::invalid_op("FlashAttention", "Q, K, V must have same shape, got Q: " + shape_str(qs) +
                                                               ", K: " + shape_str(ks) + ", V: " + shape_str(vs));
    if (qs.size() != 2)
      return BarracudaError::invalid_op("FlashAttention",
                                        "Requires 2D tensors [seq_len, head_dim], got shape: " + shape_str(qs));
    return std::nullopt;
  }
  Result<Tensor> execute() const {
    if (auto e = validate(q.shape(), k.shape(), v.shape())) return *e;
    const size_t S = q.shape()[0], D = q.shape()[1];
    return detail::sdpa(q, k, v, false, "FlashAttention", 1, 1, S, S, D);
  }
};

namespace detail {
// bch_sdpa_fwd_ex with scale 1/sqrt(D): strided operands, Hkv key/value heads.
inline std::optional<BarracudaError> sdpa_ex(const std::shared_ptr<HipDevice>& dev, const char* op, size_t B,
                                             size_t H, size_t Hkv, size_t Sq, size_t Skv, size_t D, bool causal,
                                             const Tensor& q, bch_attn_layout ql, const Tensor& k,
                                             bch_attn_layout kl, const Tensor& v, bch_attn_layout vl,
                                             const Tensor& o, bch_attn_layout ol) {
  if (auto e = check_i32(op, {B, H, Hkv, Sq, Skv, D})) return *e;
  if (B * H * Sq * D == 0) return std::nullopt;
  if (Skv == 0) return BarracudaError::invalid_op(op, "key sequence is empty (shape/dimension mismatch)");
  const float scale = 1.0f / std::sqrt((float)D);
  std::lock_guard<std::mutex> g(dev->mutex());
  return dev->check(bch_sdpa_fwd_ex(dev->ctx(), (int)B, (int)H, (int)Hkv, (int)Sq, (int)Skv, (int)D, scale,
                                    causal ? 1 : 0, q.data_ptr(), ql, k.data_ptr(), kl, v.data_ptr(), vl,
                                    o.data_ptr(), ol),
                    op);
}
inline bch_attn_layout dense_layout(size_t H, size_t S, size_t D) {
  return bch_attn_layout{(long long)(H * S * D), (long long)(S * D), (long long)D};
}
}  // namespace detail

// ops/grouped_query_attention/mod.rs:84-147: Q [B, Hq, S, D], K = V [B, Hkv, S, D],
// Hq a multiple of Hkv; query head h attends with key/value head h / (Hq / Hkv).
// One fused launch replaces the three passes of compute.rs:27-121.
struct GroupedQueryAttention {
  const Tensor& q;
  const Tensor& k;
  const Tensor& v;
  static std::optional<BarracudaError> validate(const std::vector<size_t>& qs, const std::vector<size_t>& ks,
                                                const std::vector<size_t>& vs) {
    if (qs.size() != 4 || ks.size() != 4 || vs.size() != 4)
      return BarracudaError::invalid_input("All inputs must be 4D tensors [batch, heads, seq_len, head_dim]");
    if (ks[0] != qs[0] || ks[2] != qs[2] || ks[3] != qs[3]) return BarracudaError::shape_mismatch(qs, ks);
    if (vs != ks) return BarracudaError::shape_mismatch(ks, vs);
    if (ks[1] == 0 || qs[1] % ks[1] != 0)
      return BarracudaError::invalid_input("num_q_heads (" + std::to_string(qs[1]) +
                                           ") must be divisible by num_kv_heads (" + std::to_string(ks[1]) + ")");
    return std::nullopt;
  }
  Result<Tensor> execute() const {
    if (auto e = validate(q.shape(), k.shape(), v.shape())) return *e;
    if (q.device() != k.device() || q.device() != v.device())
      return BarracudaError::device("All tensors must be on the same device");
    const auto& s = q.shape();
    const size_t B = s[0], Hq = s[1], S = s[2], D = s[3], Hkv = k.shape()[1];
    auto r = Tensor::empty(s, q.device());
    if (r.is_err()) return r;
    Tensor out = std::move(r).unwrap();
    if (auto e = detail::sdpa_ex(q.device(), "grouped_query_attention", B, Hq, Hkv, S, S, D, false, q,
                                 detail::dense_layout(Hq, S, D), k, detail::dense_layout(Hkv, S, D), v,
                                 detail::dense_layout(Hkv, S, D), out, detail::dense_layout(Hq, S, D)))
      return *e;
    return out;
  }
};

// ops/mha/mod.rs:48-187: query [B, Sq, D], key = value [B, Skv, D], four
// [D, D] weights, num_heads dividing D.  Q' = query W_q etc. (three GEMMs),
// attention per head over the [B, S, H, D/H] views of the projections (the
// reference's head_split / head_concat copies, projections.rs:18-58, become
// strides), then out = O W_o.
struct MultiHeadAttention {
  const Tensor& q;
  const Tensor& k;
  const Tensor& v;
  const Tensor& w_q;
  const Tensor& w_k;
  const Tensor& w_v;
  const Tensor& w_o;
  size_t num_heads;
  static std::optional<BarracudaError> validate(const std::vector<size_t>& qs, const std::vector<size_t>& ks,
                                                const std::vector<size_t>& vs,
                                                const std::array<std::vector<size_t>, 4>& ws, size_t heads) {
    if (qs.size() != 3 || ks.size() != 3 || vs.size() != 3) return BarracudaError::shape_mismatch(qs, {0, 0, 0});
    if (qs[0] != ks[0] || qs[0] != vs[0]) return BarracudaError::shape_mismatch(qs, ks);
    if (qs[2] != ks[2] || ks[2] != vs[2]) return BarracudaError::shape_mismatch(qs, ks);
    if (ks != vs) return BarracudaError::shape_mismatch(ks, vs);
    for (const auto& w : ws)
      if (w.size() != 2) return BarracudaError::shape_mismatch(ws[0], {0, 0});
    const size_t d = qs[2];
    for (const auto& w : ws)
      if (w != std::vector<size_t>{d, d}) return BarracudaError::shape_mismatch(ws[0], {d, d});
    if (heads == 0 || d % heads != 0)
      return BarracudaError::invalid_op("multi_head_attention", "d_model (" + std::to_string(d) +
                                                                    ") must be divisible by num_heads (" +
                                                                    std::to_string(heads) + ")");
    return std::nullopt;
  }
  Result<Tensor> execute() const {
    if (auto e = validate(q.shape(), k.shape(), v.shape(), {w_q.shape(), w_k.shape(), w_v.shape(), w_o.shape()},
                          num_heads))
      return *e;
    const size_t B = q.shape()[0], Sq = q.shape()[1], D = q.shape()[2], Skv = k.shape()[1];
    const size_t H = num_heads, hd = D / H;
    auto project = [&](const Tensor& x, size_t S, const Tensor& w) -> Result<Tensor> {
      auto x2 = x.reshape({B * S, D});
      if (x2.is_err()) return x2;
      return MatMul{x2.unwrap(), w}.execute();
    };
    auto qp = project(q, Sq, w_q);
    if (qp.is_err()) return qp;
    auto kp = project(k, Skv, w_k);
    if (kp.is_err()) return kp;
    auto vp = project(v, Skv, w_v);
    if (vp.is_err()) return vp;
    auto ro = Tensor::empty({B * Sq, D}, q.device());
    if (ro.is_err()) return ro;
    Tensor o = std::move(ro).unwrap();
    // head h of row i of batch b starts at b*S*D + i*D + h*hd
    const bch_attn_layout lq{(long long)(Sq * D), (long long)hd, (long long)D};
    const bch_attn_layout lkv{(long long)(Skv * D), (long long)hd, (long long)D};
    if (auto e = detail::sdpa_ex(q.device(), "multi_head_attention", B, H, H, Sq, Skv, hd, false, qp.unwrap(), lq,
                                 kp.unwrap(), lkv, vp.unwrap(), lkv, o, lq))
      return *e;
    auto out = MatMul{o, w_o}.execute();
    if (out.is_err()) return out;
    return out.unwrap().reshape({B, Sq, D});
  }
};

// ---------------------------------------------------------------- Tensor methods
inline Result<Tensor> Tensor::matmul(const Tensor& other) const { return MatMul{*this, other}.execute(); }
inline Result<Tensor> Tensor::matmul_ref(const Tensor& other) const { return MatMul{*this, other}.execute(); }
inline Result<Tensor> Tensor::matmul_tiled(const Tensor& other) const { return MatmulTiled{*this, other}.execute(); }
inline Result<Tensor> Tensor::batch_matmul(const Tensor& other) const { return BatchMatMul{*this, other}.execute(); }
inline Result<Tensor> Tensor::softmax() const { return Softmax{*this}.execute(); }
inline Result<Tensor> Tensor::relu() const { return ReLU{*this}.execute(); }
inline Result<Tensor> Tensor::gelu_wgsl() const { return GELU{*this}.execute(); }
inline Result<Tensor> Tensor::layer_norm_wgsl(float epsilon) const { return LayerNorm{*this, epsilon}.execute(); }
inline Result<Tensor> Tensor::softmax_dim(size_t axis) const {
  if (auto e = validate_softmax_dim(shape_, axis)) return *e;
  auto r = Tensor::empty(shape_, dev_);
  if (r.is_err() || len() == 0) return r;
  Tensor out = std::move(r).unwrap();
  size_t outer = 1, inner = 1;
  for (size_t i = 0; i < axis; ++i) outer *= shape_[i];
  for (size_t i = axis + 1; i < shape_.size(); ++i) inner *= shape_[i];
  std::lock_guard<std::mutex> g(dev_->mutex());
  if (auto e = dev_->check(bch_softmax_axis(dev_->ctx(), (long long)outer, (long long)shape_[axis], (long long)inner,
                                            data_ptr(), out.data_ptr()),
                           "softmax_dim"))
    return *e;
  return out;
}
inline Result<Tensor> Tensor::attention(const Tensor& key, const Tensor& value) const {
  return Attention{*this, key, value}.execute();
}
inline Result<Tensor> Tensor::scaled_dot_product_attention(const Tensor& key, const Tensor& value) const {
  return ScaledDotProductAttention{*this, key, value}.execute();
}
inline Result<Tensor> Tensor::causal_attention(const Tensor& key, const Tensor& value) const {
  return CausalAttention{*this, key, value}.execute();
}
inline Result<Tensor> Tensor::grouped_query_attention(const Tensor& key, const Tensor& value) const {
  return GroupedQueryAttention{*this, key, value}.execute();
}
inline Result<Tensor> Tensor::multi_head_attention(const Tensor& key, const Tensor& value, const Tensor& w_q,
                                                   const Tensor& w_k, const Tensor& w_v, const Tensor& w_o,
                                                   size_t num_heads) const {
  return MultiHeadAttention{*this, key, value, w_q, w_k, w_v, w_o, num_heads}.execute();
}

// ---------------------------------------------------------------- nn
namespace nn {
// nn/fused_mlp.rs:25-31 (ReLU); GELU applies gelu_f64.wgsl's tanh form in the
// same GEMM epilogue
enum class Activation { ReLU, GELU };

// nn/fused_mlp.rs:38-168: per layer y = relu(x W^T + b) (W [out, in]) or
// relu(x W + b) (W [in, out]); the reference dispatches linear_f64.wgsl and
// relu_f64.wgsl per layer, here each layer is one GEMM whose epilogue adds
// the bias and applies ReLU (bch_sgemm_ex).  Same validation order and
// messages.  Non-square [in, out] weights: the reference's shader still
// indexes them as [out, in] (linear_f64.wgsl:35); this computes x W.
inline Result<Tensor> fused_mlp(const Tensor& input, const std::vector<Tensor>& weights,
                                const std::vector<Tensor>& biases, Activation activation = Activation::ReLU) {
  if (weights.size() != biases.size())
    return BarracudaError::invalid_input("fused_mlp: weights len " + std::to_string(weights.size()) +
                                         " != biases len " + std::to_string(biases.size()));
  if (weights.empty()) return BarracudaError::invalid_input("fused_mlp: at least one layer required");
  const auto& shape = input.shape();
  if (shape.size() != 2)
    return BarracudaError::invalid_input("fused_mlp: input must be 2D, got " + shape_str(shape));
  const size_t batch = shape[0];
  size_t in_features = shape[1];
  struct Layer {
    size_t in, out;
    int transb;
  };
  std::vector<Layer> layers;
  for (size_t i = 0; i < weights.size(); ++i) {
    const auto& ws = weights[i].shape();
    Layer L{};
    if (ws.size() != 2)
      return BarracudaError::invalid_input("fused_mlp: weight[" + std::to_string(i) + "] must be 2D");
    if (ws[1] == in_features)
      L = {ws[1], ws[0], 1};
    else if (ws[0] == in_features)
      L = {ws[0], ws[1], 0};
    else
      return BarracudaError::invalid_input("fused_mlp: weight[" + std::to_string(i) + "] shape " + shape_str(ws) +
                                           " incompatible");
    if (biases[i].shape() != std::vector<size_t>{L.out})
      return BarracudaError::invalid_input("fused_mlp: bias[" + std::to_string(i) + "] shape mismatch");
    layers.push_back(L);
    in_features = L.out;
  }
  auto dev = input.device();
  const int act = activation == Activation::ReLU ? BCH_ACT_RELU : BCH_ACT_GELU;
  Tensor x = input;
  for (size_t i = 0; i < layers.size(); ++i) {
    const Layer& L = layers[i];
    if (auto e = detail::check_i32("fused_mlp", {batch, L.in, L.out})) return *e;
    auto r = Tensor::empty({batch, L.out}, dev);
    if (r.is_err()) return r;
    Tensor y = std::move(r).unwrap();
    if (batch != 0 && L.out != 0) {
      const int lin = L.in > 1 ? (int)L.in : 1, lout = L.out > 1 ? (int)L.out : 1;
      std::lock_guard<std::mutex> g(dev->mutex());
      if (auto e = dev->check(bch_sgemm_ex(dev->ctx(), L.transb, (int)batch, (int)L.out, (int)L.in, x.data_ptr(),
                                           lin, weights[i].data_ptr(), L.transb ? lin : lout,
                                           biases[i].data_ptr(), act, y.data_ptr(), lout),
                              "fused_mlp"))
        return *e;
    }
    x = y;
  }
  return x;
}
}  // namespace nn

// ---------------------------------------------------------------- f64 GEMM
// ops/linalg/gemm_f64.rs:77-249: batched C = alpha op(A) op(B) + beta C over
// packed row-major f64 host data (the reference's C buffer starts zeroed, so
// beta multiplies zero).  One bch_dgemm on the FP64 matrix cores.
struct GemmF64 {
  static Result<std::vector<double>> execute(const std::shared_ptr<HipDevice>& dev, const std::vector<double>& a,
                                             const std::vector<double>& b, size_t m, size_t k, size_t n,
                                             size_t batch_size) {
    return execute_gemm(dev, a, b, m, k, n, batch_size, 1.0, 0.0);
  }
  static Result<std::vector<double>> execute_gemm(const std::shared_ptr<HipDevice>& dev,
                                                  const std::vector<double>& a, const std::vector<double>& b,
                                                  size_t m, size_t k, size_t n, size_t batch_size, double alpha,
                                                  double beta) {
    return execute_gemm_ex(dev, a, b, m, k, n, batch_size, alpha, beta, false, false);
  }
  static Result<std::vector<double>> execute_gemm_ex(const std::shared_ptr<HipDevice>& dev,
                                                     const std::vector<double>& a, const std::vector<double>& b,
                                                     size_t m, size_t k, size_t n, size_t batch_size, double alpha,
                                                     double beta, bool trans_a, bool trans_b) {
    const size_t ea = batch_size * m * k, eb = batch_size * k * n;
    if (a.size() != ea)
      return BarracudaError::invalid_input("A: expected " + std::to_string(ea) + " elements, got " +
                                           std::to_string(a.size()));
    if (b.size() != eb)
      return BarracudaError::invalid_input("B: expected " + std::to_string(eb) + " elements, got " +
                                           std::to_string(b.size()));
    std::vector<double> c(batch_size * m * n, 0.0);
    if (auto e = run(dev, a, b, c, m, k, n, batch_size, alpha, beta, trans_a, trans_b)) return *e;
    return c;
  }

  // upload a and b, run bch_dgemm with c as the initial C, read C back into c
  static std::optional<BarracudaError> run(const std::shared_ptr<HipDevice>& dev, const std::vector<double>& a,
                                           const std::vector<double>& b, std::vector<double>& c, size_t m, size_t k,
                                           size_t n, size_t batch, double alpha, double beta, bool ta, bool tb) {
    if (auto e = detail::check_i32("gemm_f64", {batch, m, n, k})) return e;
    if (c.empty()) return std::nullopt;
    std::lock_guard<std::mutex> g(dev->mutex());
    void *pa = nullptr, *pb = nullptr, *pc = nullptr;
    std::optional<BarracudaError> err;
    auto chk = [&](bch_status st, const char* op) {
      if (!err) err = dev->check(st, op);
      return !err;
    };
    if (chk(bch_alloc(dev->ctx(), a.size() * 8, &pa), "alloc_buffer") &&
        chk(bch_alloc(dev->ctx(), b.size() * 8, &pb), "alloc_buffer") &&
        chk(bch_alloc(dev->ctx(), c.size() * 8, &pc), "alloc_buffer") &&
        (a.empty() || chk(bch_upload(dev->ctx(), pa, a.data(), a.size() * 8), "upload")) &&
        (b.empty() || chk(bch_upload(dev->ctx(), pb, b.data(), b.size() * 8), "upload")) &&
        chk(bch_upload(dev->ctx(), pc, c.data(), c.size() * 8), "upload")) {
      const int lda = (int)std::max<size_t>(ta ? m : k, 1), ldb = (int)std::max<size_t>(tb ? k : n, 1);
      if (chk(bch_dgemm(dev->ctx(), ta, tb, (int)batch, (int)m, (int)n, (int)k, alpha, static_cast<double*>(pa), lda,
                        (long long)(m * k), static_cast<double*>(pb), ldb, (long long)(k * n), beta,
                        static_cast<double*>(pc), (int)std::max<size_t>(n, 1), (long long)(m * n)),
              "gemm_f64"))
        chk(bch_download(dev->ctx(), c.data(), pc, c.size() * 8), "download");
    }
    for (void* p : {pa, pb, pc})
      if (p) bch_free(dev->ctx(), p);
    return err;
  }
};

// ops/linalg/gemm_f64.rs:252-456: B held on the device, C = A B for many A
// (the reference's dispatch swaps its m and n grid dimensions; here every
// element is computed whatever m and n are).
class GemmCachedF64 {
 public:
  static Result<GemmCachedF64> create(std::shared_ptr<HipDevice> dev, const std::vector<double>& b, size_t k,
                                      size_t n, size_t batch_size) {
    if (b.size() != batch_size * k * n)
      return BarracudaError::invalid_input("GemmCachedF64: B has " + std::to_string(b.size()) +
                                           " elements, expected batch×K×N=" + std::to_string(batch_size * k * n));
    return GemmCachedF64(std::move(dev), b, k, n, batch_size);
  }
  Result<std::vector<double>> multiply(const std::vector<double>& a, size_t m) const {
    if (a.size() != batch_size * m * k)
      return BarracudaError::invalid_input("GemmCachedF64::execute_to_buffer: A has " + std::to_string(a.size()) +
                                           " elements, expected batch×M×K=" + std::to_string(batch_size * m * k));
    std::vector<double> c(batch_size * m * n, 0.0);
    if (auto e = GemmF64::run(dev_, a, b_, c, m, k, n, batch_size, 1.0, 0.0, false, false)) return *e;
    return c;
  }
  size_t k, n, batch_size;

 private:
  GemmCachedF64(std::shared_ptr<HipDevice> dev, std::vector<double> b, size_t k_, size_t n_, size_t batch)
      : k(k_), n(n_), batch_size(batch), dev_(std::move(dev)), b_(std::move(b)) {}
  std::shared_ptr<HipDevice> dev_;
  std::vector<double> b_;
};

// ---------------------------------------------------------------- session
// The unit value of Result<()>.
struct Unit {};

// session/mod.rs:60-99: the [B, H, S, D] dimensions of an attention op.
struct AttentionDims {
  size_t batch_size = 0;
  size_t n_heads = 0;
  size_t seq_len = 0;
  size_t head_dim = 0;
  size_t total_elements() const { return batch_size * n_heads * seq_len * head_dim; }
  // (batch_size, seq_len, n_heads, head_dim), each checked to fit u32
  // (cast.rs:31-37 usize_as_u32)
  Result<std::array<uint32_t, 4>> as_u32() const {
    const size_t v[4] = {batch_size, seq_len, n_heads, head_dim};
    std::array<uint32_t, 4> out{};
    for (int i = 0; i < 4; ++i) {
      if (v[i] > (size_t)UINT32_MAX) return BarracudaError::cast_overflow("usize", "u32", std::to_string(v[i]));
      out[i] = (uint32_t)v[i];
    }
    return out;
  }
};

class TensorSession;

// session/tensor.rs:14-68: a buffer owned by a session, with its shape.  The
// buffer exists from creation; an op's output reads as zeros until
// TensorSession::run() has executed the op.
class SessionTensor {
 public:
  const std::vector<size_t>& shape() const { return shape_; }
  size_t len() const { return detail::numel(shape_); }
  bool is_empty() const { return len() == 0; }
  size_t buffer_id() const { return id_; }
  Result<std::vector<float>> to_vec() const {
    std::vector<float> out(len());
    if (!out.empty()) {
      std::lock_guard<std::mutex> g(buf_->dev->mutex());
      if (auto e = buf_->dev->check(
              bch_download(buf_->dev->ctx(), out.data(), buf_->ptr, out.size() * sizeof(float)), "download"))
        return *e;
    }
    return out;
  }
  // a standalone Tensor holding a copy (tensor.rs:64-67)
  Result<Tensor> to_tensor() const {
    auto v = to_vec();
    if (v.is_err()) return v.error();
    return Tensor::from_data(v.value(), shape_, buf_->dev);
  }

 private:
  friend class TensorSession;
  SessionTensor(const void* owner, size_t id, std::shared_ptr<detail::DeviceBuffer> b, std::vector<size_t> s)
      : owner_(owner), id_(id), buf_(std::move(b)), shape_(std::move(s)) {}
  const void* owner_;
  size_t id_;
  std::shared_ptr<detail::DeviceBuffer> buf_;
  std::vector<size_t> shape_;
};

// session/mod.rs:118-540: ops are recorded, then run() enqueues them all, in
// order, on the device's one stream and waits once.  Outputs are allocated
// (zero-filled) when an op is recorded.  Routed to this library's kernels
// with grids that cover the whole problem, so the reference session's
// dispatch defects (partial non-square matmul tiers, session/types.rs:53-58;
// a one-workgroup softmax, dispatch.rs:217; an attention grid over the
// 65,535 limit, dispatch.rs:289-295) are not reproduced.  softmax is the
// global softmax over every element, what the reference session's shader
// computes for each output it writes; attention is non-causal.
class TensorSession {
 public:
  explicit TensorSession(std::shared_ptr<HipDevice> dev) : dev_(std::move(dev)) {}
  static TensorSession with_device(std::shared_ptr<HipDevice> dev) { return TensorSession(std::move(dev)); }
  TensorSession(const TensorSession&) = delete;
  TensorSession& operator=(const TensorSession&) = delete;
  TensorSession(TensorSession&&) = delete;

  // session/mod.rs:155-165
  void reset() {
    ops_.clear();
    executed_ = false;
  }
  size_t num_ops() const { return ops_.size(); }
  bool executed() const { return executed_; }

  // session/mod.rs:172-198
  Result<SessionTensor> tensor(const std::vector<float>& data) { return tensor_with_shape(data, {data.size()}); }
  Result<SessionTensor> tensor_with_shape(const std::vector<float>& data, const std::vector<size_t>& shape) {
    if (data.size() != detail::numel(shape)) return BarracudaError::invalid_shape(shape, {data.size()});
    auto b = alloc(shape, false);
    if (b.is_err()) return b.error();
    if (!data.empty()) {
      std::lock_guard<std::mutex> g(dev_->mutex());
      if (auto e = dev_->check(bch_upload(dev_->ctx(), b.value()->ptr, data.data(), data.size() * sizeof(float)),
                               "upload"))
        return *e;
    }
    return reg(std::move(b).unwrap(), shape);
  }
  // session/mod.rs:204-207: the copy stays in HBM (device to device) instead
  // of the reference's read-back and re-upload; the result is the same.
  Result<SessionTensor> import(const Tensor& t) {
    if (t.device() != dev_) {
      auto v = t.to_vec();
      if (v.is_err()) return v.error();
      return tensor_with_shape(v.value(), t.shape());
    }
    auto b = alloc(t.shape(), false);
    if (b.is_err()) return b.error();
    if (b.value()->bytes) {
      std::lock_guard<std::mutex> g(dev_->mutex());
      if (auto e = dev_->check(bch_copy(dev_->ctx(), b.value()->ptr, t.data_ptr(), b.value()->bytes), "import"))
        return *e;
    }
    return reg(std::move(b).unwrap(), t.shape());
  }

  // session/mod.rs:305-333: output[m x n] = a[m x k] b[k x n]
  Result<SessionTensor> matmul(const SessionTensor& a, const SessionTensor& b) {
    if (auto e = own({&a, &b})) return *e;
    if (a.shape().size() != 2 || b.shape().size() != 2) return BarracudaError::invalid_shape(a.shape(), b.shape());
    const size_t m = a.shape()[0], k = a.shape()[1];
    if (b.shape()[0] != k) return BarracudaError::shape_mismatch({m, k}, b.shape());
    const size_t n = b.shape()[1];
    for (size_t d : {m, k, n})  // session/mod.rs:327-329 usize_as_u32
      if (d > (size_t)UINT32_MAX) return BarracudaError::cast_overflow("usize", "u32", std::to_string(d));
    if (auto e = detail::check_i32("matmul", {m, k, n})) return *e;
    auto out = alloc_output({m, n});
    if (out.is_ok()) ops_.push_back({Op::MatMul, {a.id_, b.id_, out.value().id_, 0}, {m, k, n, 0}});
    return out;
  }

  // session/mod.rs:364-371, over every element (dispatch.rs:211)
  Result<SessionTensor> softmax(const SessionTensor& a) {
    if (auto e = own({&a})) return *e;
    auto out = alloc_output(a.shape());
    if (out.is_ok()) ops_.push_back({Op::Softmax, {a.id_, out.value().id_, 0, 0}, {a.len(), 0, 0, 0}});
    return out;
  }

  // session/mod.rs:423-446: [B, S, H*D] -> [B, H, S, D] (head_split_f64.wgsl)
  Result<SessionTensor> head_split(const SessionTensor& a, const AttentionDims& dims) {
    return head_permute(false, a, dims);
  }
  // session/mod.rs:451-480: [B, H, S, D] -> [B, S, H*D] (head_concat_f64.wgsl)
  Result<SessionTensor> head_concat(const SessionTensor& a, const AttentionDims& dims) {
    return head_permute(true, a, dims);
  }

  // session/mod.rs:481-518: softmax(Q K^T / sqrt(D)) V over [B, H, S, D]
  Result<SessionTensor> attention(const SessionTensor& q, const SessionTensor& k, const SessionTensor& v,
                                  const AttentionDims& dims) {
    if (auto e = own({&q, &k, &v})) return *e;
    const size_t expected = dims.total_elements();
    const std::pair<const char*, const SessionTensor*> qkv[3] = {{"q", &q}, {"k", &k}, {"v", &v}};
    for (const auto& [name, t] : qkv)
      if (t->len() != expected)
        return BarracudaError::invalid_input(std::string("attention: ") + name + " len " + std::to_string(t->len()) +
                                             " ≠ B×H×S×D=" + std::to_string(expected));
    if (auto e = dims.as_u32(); e.is_err()) return e.error();
    if (auto e = detail::check_i32("attention", {dims.batch_size, dims.n_heads, dims.seq_len, dims.head_dim}))
      return *e;
    auto out = alloc_output({dims.batch_size, dims.n_heads, dims.seq_len, dims.head_dim});
    if (out.is_ok())
      ops_.push_back({Op::Attention, {q.id_, k.id_, v.id_, out.value().id_},
                      {dims.batch_size, dims.n_heads, dims.seq_len, dims.head_dim}});
    return out;
  }

  // session/mod.rs:521-540: every recorded op, in order, one wait.  A launch
  // error stops the batch; ops enqueued before it have been submitted.
  Result<Unit> run() {
    if (ops_.empty()) return Unit{};
    std::lock_guard<std::mutex> g(dev_->mutex());
    bch_ctx* c = dev_->ctx();
    auto p = [this](size_t id) { return static_cast<float*>(bufs_[id]->ptr); };
    for (const Op& op : ops_) {
      bch_status st = BCH_OK;
      const char* name = "run";
      switch (op.kind) {
        case Op::MatMul: {
          const int m = (int)op.dim[0], k = (int)op.dim[1], n = (int)op.dim[2];
          const int lk = k > 1 ? k : 1, ln = n > 1 ? n : 1;
          name = "matmul";
          if (m && n) st = bch_sgemm(c, m, n, k, p(op.buf[0]), lk, p(op.buf[1]), ln, p(op.buf[2]), ln);
          break;
        }
        case Op::Softmax:
          name = "softmax";
          if (op.dim[0]) st = bch_softmax_rows(c, 1, (long long)op.dim[0], p(op.buf[0]), p(op.buf[1]));
          break;
        case Op::Attention: {
          const size_t B = op.dim[0], H = op.dim[1], S = op.dim[2], D = op.dim[3];
          name = "attention";
          if (B * H * S * D != 0)
            st = bch_sdpa_fwd(c, (int)B, (int)H, (int)S, (int)S, (int)D, 1.0f / std::sqrt((float)D), 0,
                              p(op.buf[0]), p(op.buf[1]), p(op.buf[2]), p(op.buf[3]));
          break;
        }
        case Op::HeadSplit:
        case Op::HeadConcat: {
          const size_t B = op.dim[0], S = op.dim[1], H = op.dim[2], D = op.dim[3];
          const bool concat = op.kind == Op::HeadConcat;
          name = concat ? "head_concat" : "head_split";
          if (B * S * H * D != 0)
            st = (concat ? bch_head_concat : bch_head_split)(c, (int)B, (int)S, (int)H, (int)D, p(op.buf[0]),
                                                              p(op.buf[1]));
          break;
        }
      }
      if (auto e = dev_->check(st, name)) return *e;
    }
    if (auto e = dev_->check(bch_sync(c), "run")) return *e;
    executed_ = true;
    return Unit{};
  }

 private:
  struct Op {
    enum Kind { MatMul, Softmax, Attention, HeadSplit, HeadConcat } kind;
    size_t buf[4];
    size_t dim[4];
  };

  Result<SessionTensor> head_permute(bool concat, const SessionTensor& a, const AttentionDims& dims) {
    if (auto e = own({&a})) return *e;
    const char* op = concat ? "head_concat" : "head_split";
    const size_t expected = dims.total_elements();
    if (a.len() != expected)
      return BarracudaError::invalid_input(std::string(op) + ": input len " + std::to_string(a.len()) + " ≠ " +
                                           (concat ? "B×H×S×D=" : "B×S×H×D=") + std::to_string(expected));
    if (auto e = dims.as_u32(); e.is_err()) return e.error();
    if (auto e = detail::check_i32(op, {dims.batch_size, dims.n_heads, dims.seq_len, dims.head_dim,
                                        dims.seq_len * dims.head_dim, dims.n_heads * dims.head_dim}))
      return *e;
    auto out = concat ? alloc_output({dims.batch_size, dims.seq_len, dims.n_heads * dims.head_dim})
                      : alloc_output({dims.batch_size, dims.n_heads, dims.seq_len, dims.head_dim});
    if (out.is_ok())
      ops_.push_back({concat ? Op::HeadConcat : Op::HeadSplit, {a.id_, out.value().id_, 0, 0},
                      {dims.batch_size, dims.seq_len, dims.n_heads, dims.head_dim}});
    return out;
  }

  Result<std::shared_ptr<detail::DeviceBuffer>> alloc(const std::vector<size_t>& shape, bool zero) {
    auto buf = std::make_shared<detail::DeviceBuffer>();
    buf->dev = dev_;
    buf->bytes = detail::numel(shape) * sizeof(float);
    if (buf->bytes) {
      std::lock_guard<std::mutex> g(dev_->mutex());
      if (auto e = dev_->check(bch_alloc(dev_->ctx(), buf->bytes, &buf->ptr), "alloc_buffer")) return *e;
      if (zero)
        if (auto e = dev_->check(bch_memset(dev_->ctx(), buf->ptr, 0, buf->bytes), "alloc_output")) return *e;
    }
    return buf;
  }
  SessionTensor reg(std::shared_ptr<detail::DeviceBuffer> b, const std::vector<size_t>& shape) {
    bufs_.push_back(b);
    return SessionTensor(this, bufs_.size() - 1, std::move(b), shape);
  }
  Result<SessionTensor> alloc_output(const std::vector<size_t>& shape) {
    auto b = alloc(shape, true);
    if (b.is_err()) return b.error();
    return reg(std::move(b).unwrap(), shape);
  }
  std::optional<BarracudaError> own(std::initializer_list<const SessionTensor*> ts) const {
    for (const SessionTensor* t : ts)
      if (t->owner_ != this) return BarracudaError::invalid_input("session tensor belongs to another TensorSession");
    return std::nullopt;
  }

  std::shared_ptr<HipDevice> dev_;
  std::vector<std::shared_ptr<detail::DeviceBuffer>> bufs_;
  std::vector<Op> ops_;
  bool executed_ = false;
};

}  // namespace barracuda
