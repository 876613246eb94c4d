// vearo_backend.h -- host-side mirror of vearo's BackendOps plugin interface for
// the HIP backend, written in C++ above the C ABI of libvearo_hip.so.
//
// The reference registers per-device op tables (crates/vearo-core/src/tensor.rs:1108-1196)
// that take `&Tensor` and return fresh contiguous tensors; this header restates
// that surface -- the same slot names, argument meaning and panic messages -- so
// the backend can be exercised end to end (tests/cpp) the way the reference's
// own tests drive its CUDA backend (crates/vearo-backend-cuda/src/lib.rs:1638-1826).
// A Rust `vearo-backend-hip` crate would fill the same table with thin wrappers
// over the extern "C" entry points used here.
#pragma once
#include <array>
#include <cstdint>
#include <initializer_list>
#include <memory>
#include <stdexcept>
#include <string>
#include <tuple>
#include <vector>

namespace vearo_hip {

constexpr int MAX_RANK = 8;      // vearo-core shape.rs:2
constexpr int NUM_BACKENDS = 4;  // vearo-core device.rs:5

// A panic of the reference (assert!/expect) carrying the same message text.
struct Panic : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// An std::io::Error the reference would return (a file that cannot be
// created, opened, read or written, or ends early).
struct IoError : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// Device with the backend slot the reference reserves for a third backend
// (device.rs:1-5: 0 = CPU, 1 = CUDA, 2/3 reserved).
struct Device {
  enum Kind { Cpu, Cuda, Hip } kind = Hip;
  int index = 0;
  static Device hip(int i = 0) { return {Hip, i}; }
  int backend_idx() const { return kind == Cpu ? 0 : kind == Cuda ? 1 : 2; }
  bool operator==(const Device& o) const { return kind == o.kind && index == o.index; }
};

// Rank <= 8 dims (shape.rs:8-12).
struct Shape {
  int rank = 0;
  std::array<int64_t, MAX_RANK> d{};
  Shape() = default;
  Shape(std::initializer_list<int64_t> dims);
  explicit Shape(const std::vector<int64_t>& dims);
  int64_t operator[](int i) const { return d[i]; }
  int64_t numel() const;
  Shape contiguous_strides() const;
  std::vector<int64_t> dims() const { return std::vector<int64_t>(d.begin(), d.begin() + rank); }
  bool operator==(const Shape& o) const;
  bool operator!=(const Shape& o) const { return !(*this == o); }
  std::string str() const;
};

// Device storage: one arena block, released to the arena when the last view goes.
struct Storage {
  void* ptr = nullptr;
  size_t bytes = 0;
  ~Storage();
};

class Tensor {
 public:
  Tensor() = default;
  // Zero-filled device tensor (Tensor::zeros_on, tensor.rs:88-117).
  static Tensor zeros(const Shape& s, Device dev = Device::hip());
  // Uninitialised device tensor for op outputs every kernel fully overwrites.
  static Tensor empty(const Shape& s, Device dev = Device::hip());
  // Host data to device (Tensor::from_f32 + to(device), tensor.rs:184-219).
  static Tensor from_f32(const std::vector<float>& data, const Shape& s, Device dev = Device::hip());

  const Shape& shape() const { return shape_; }
  const Shape& strides() const { return strides_; }
  Device device() const { return device_; }
  bool is_contiguous() const;
  const float* data() const { return static_cast<const float*>(storage_->ptr); }
  float* data() { return static_cast<float*>(storage_->ptr); }
  const void* storage_id() const { return storage_.get(); }
  long use_count() const { return storage_.use_count(); }

  // Views (tensor.rs:493-620) and the device-side contiguous copy.
  Tensor transpose(int a, int b) const;
  Tensor permute(const std::vector<int>& axes) const;
  Tensor reshape(const Shape& s) const;
  Tensor contiguous() const;
  // Synchronous read-back; reports any deferred device panic first.
  std::vector<float> to_vec_f32() const;

  // Dispatching op methods (tensor.rs:1371-1751): look up BACKEND_OPS by device.
  Tensor add(const Tensor& o) const;
  Tensor sub(const Tensor& o) const;
  Tensor mul(const Tensor& o) const;
  Tensor div(const Tensor& o) const;
  Tensor sum(size_t dim, bool keep_dim) const;
  Tensor mean(size_t dim, bool keep_dim) const;
  Tensor gelu() const;
  Tensor softmax(size_t dim) const;
  Tensor layernorm(const Tensor& w, const Tensor& b, float eps) const;
  std::tuple<Tensor, Tensor, Tensor> layernorm_backward(const Tensor& w, const Tensor& b,
                                                        const Tensor& grad_out, float eps) const;
  Tensor embedding(const Tensor& weight) const;
  Tensor embedding_backward(const Tensor& weight, const Tensor& grad_out) const;
  Tensor cross_entropy(const Tensor& targets) const;
  Tensor cross_entropy_backward(const Tensor& targets, const Tensor& grad_out) const;
  Tensor matmul(const Tensor& o) const;
  Tensor fused_attention(const Tensor& k, const Tensor& v, const Tensor* mask) const;
  std::tuple<Tensor, Tensor, Tensor> fused_attention_backward(const Tensor& k, const Tensor& v,
                                                              const Tensor* mask,
                                                              const Tensor& grad_out) const;

 private:
  std::shared_ptr<Storage> storage_;
  Shape shape_, strides_;
  Device device_;
  friend Tensor make_view(const Tensor&, const Shape&, const Shape&);
};

using BinaryOpFn = Tensor (*)(const Tensor&, const Tensor&);
using UnaryOpFn = Tensor (*)(const Tensor&);
using ReduceOpFn = Tensor (*)(const Tensor&, size_t, bool);

// The 26 slots of tensor.rs:1108-1175, same names and order.
struct BackendOps {
  BinaryOpFn add, sub, mul, div, matmul;
  UnaryOpFn relu;
  ReduceOpFn sum, mean;
  UnaryOpFn gelu;
  Tensor (*softmax)(const Tensor&, size_t);
  Tensor (*layernorm)(const Tensor&, const Tensor&, const Tensor&, float);
  std::tuple<Tensor, Tensor, Tensor> (*layernorm_backward)(const Tensor&, const Tensor&, const Tensor&,
                                                           const Tensor&, float);
  Tensor (*embedding)(const Tensor&, const Tensor&);
  Tensor (*embedding_backward)(const Tensor&, const Tensor&, const Tensor&);
  Tensor (*cross_entropy)(const Tensor&, const Tensor&);
  Tensor (*cross_entropy_backward)(const Tensor&, const Tensor&, const Tensor&);
  Tensor (*conv2d)(const Tensor&, const Tensor&, const Tensor&, size_t, size_t);
  std::tuple<Tensor, Tensor, Tensor> (*conv2d_backward)(const Tensor&, const Tensor&, const Tensor&, size_t,
                                                        size_t);
  Tensor (*maxpool2d)(const Tensor&, size_t, size_t, size_t);
  Tensor (*maxpool2d_backward)(const Tensor&, const Tensor&, size_t, size_t, size_t);
  Tensor (*avgpool2d)(const Tensor&, size_t, size_t, size_t);
  Tensor (*avgpool2d_backward)(const Tensor&, const Tensor&, size_t, size_t, size_t);
  Tensor (*batchnorm)(const Tensor&, const Tensor&, const Tensor&, const Tensor&, const Tensor&, bool, float,
                      float);
  std::tuple<Tensor, Tensor, Tensor> (*batchnorm_backward)(const Tensor&, const Tensor&, const Tensor&,
                                                           const Tensor&, const Tensor&, const Tensor&, bool,
                                                           float);
  Tensor (*fused_attention)(const Tensor&, const Tensor&, const Tensor&, const Tensor*);
  std::tuple<Tensor, Tensor, Tensor> (*fused_attention_backward)(const Tensor&, const Tensor&, const Tensor&,
                                                                 const Tensor*, const Tensor&);
};

// register_backend_ops / get_backend_ops (tensor.rs:1181-1196): first
// registration wins, so repeated init() calls are harmless.
void register_backend_ops(Device device, const BackendOps& ops);
const BackendOps* get_backend_ops(Device device);

// vearo_backend_hip::init(): vh_init on the device, then register the table.
void init(int device = 0);
// The HIP backend's table (what init registers).
BackendOps hip_backend_ops();
// Wait for queued work; throws Panic for a deferred device panic.
void synchronize();

// The autograd arms on the hot path (crates/vearo-autograd/src/lib.rs:542-553),
// composed from BackendOps calls exactly as the arms compose them.
Tensor softmax_backward_arm(const Tensor& x, const Tensor& grad_out, size_t dim);
// The same arm as one fused launch (vh_softmax_bwd).
Tensor softmax_backward_fused(const Tensor& x, const Tensor& grad_out);
// Gelu arm with the mask built on the device: grad_out * gelu'(x).
Tensor gelu_backward_fused(const Tensor& x, const Tensor& grad_out);

// vearo::checkpoint (crates/vearo/src/checkpoint.rs:9-91) for device tensors:
// the same `.ve` file, the same panics (Panic) and io errors (IoError).
// load_checkpoint writes into the tensors' storage, as copy_from_slice does.
void save_checkpoint(const std::vector<Tensor>& params, const std::string& path);
void load_checkpoint(const std::vector<Tensor>& params, const std::string& path);

}  // namespace vearo_hip
