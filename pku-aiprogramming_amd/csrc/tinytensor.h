// TinyTensor<T>: the drop-in tensor of the `myTensor` module, rebuilt on the
// MI355X C-ABI (include/tt_attn.h) instead of direct CUDA runtime calls.
//
// Same public fields and methods as the reference class
// (Task3/Tinytensor/src/TinyTensor.h:11-76): shape, device ("cpu"/"gpu"),
// p_data, size; constructors from (shape, device), (shape, device, data),
// (numpy array, device) and copy; Size, +, -, [], get_shape, get_device,
// get_data, flatten, cpu, gpu, random, zeros, ones, negative, mults, floatks,
// resize, Relu/Sigmoid Forward/Backward and operator<<.
//
// Differences by design: device storage comes from the library's caching
// allocator (tt_malloc), work is ordered on one HIP stream and host-visible
// copies wait for it, every HIP failure raises std::runtime_error, sizes are
// 64-bit, and a bf16 storage type (TinyTensor<bf16>) is added for the
// attention path.  numpy() returns the data as an ndarray in one copy.
#pragma once

#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>

#include <cstdint>
#include <cstring>
#include <ostream>
#include <string>
#include <vector>

#include "../../include/tt_attn.h"

// bfloat16 storage element.  Host values are float; conversion rounds to
// nearest even (NaN stays NaN).
struct bf16 {
  uint16_t bits;
};

inline uint16_t float_to_bf16_bits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}
inline float bf16_bits_to_float(uint16_t b) {
  uint32_t u = uint32_t(b) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// Storage type -> host value type, C-ABI dtype code and conversions.
template <typename T> struct Dtype {
  using host = T;
  static host to_host(T v) { return v; }
  static T from_host(host v) { return v; }
};
template <> struct Dtype<float> {
  using host = float;
  static constexpr int code = TT_F32;
  static constexpr const char* name = "float";
  static host to_host(float v) { return v; }
  static float from_host(host v) { return v; }
};
template <> struct Dtype<double> {
  using host = double;
  static constexpr int code = TT_F64;
  static constexpr const char* name = "double";
  static host to_host(double v) { return v; }
  static double from_host(host v) { return v; }
};
template <> struct Dtype<int> {
  using host = int;
  static constexpr int code = TT_I32;
  static constexpr const char* name = "int";
  static host to_host(int v) { return v; }
  static int from_host(host v) { return v; }
};
template <> struct Dtype<bf16> {
  using host = float;
  static constexpr int code = TT_BF16;
  static constexpr const char* name = "bf16";
  static host to_host(bf16 v) { return bf16_bits_to_float(v.bits); }
  static bf16 from_host(host v) { return bf16{float_to_bf16_bits(v)}; }
};

// Throws std::runtime_error with tt_last_error() when rc != TT_OK
// (std::invalid_argument for TT_ERR_ARG / TT_ERR_UNSUPPORTED).
void tt_check(int rc, const char* what);

template <typename Type = float>
class TinyTensor {
 public:
  using Host = typename Dtype<Type>::host;

  std::vector<int> shape;
  std::string device;
  Type* p_data = nullptr;
  size_t size = 0;

  TinyTensor(const std::vector<int>& shape, const std::string& device);
  TinyTensor(const std::vector<int>& shape, const std::string& device, const std::vector<Host>& data);
  TinyTensor(const pybind11::array_t<Host>& data, const std::string& device);
  TinyTensor(const TinyTensor<Type>& other);
  ~TinyTensor();

  size_t Size() const;

  TinyTensor<Type>& operator=(const TinyTensor<Type>& other);
  TinyTensor<Type> operator+(const TinyTensor<Type>& other) const;
  TinyTensor<Type> operator-(const TinyTensor<Type>& other) const;
  TinyTensor<Type> operator[](int index) const;

  std::vector<int> get_shape() const;
  std::string get_device() const;
  std::vector<Host> get_data() const;
  pybind11::array_t<Host> numpy() const;
  TinyTensor<Type> flatten() const;

  TinyTensor<Type>& cpu();
  TinyTensor<Type>& gpu();
  TinyTensor<Type>& random(Host a, Host b);
  TinyTensor<Type>& zeros();
  TinyTensor<Type>& ones();
  TinyTensor<Type>& negative();
  TinyTensor<Type>& mults(Host scalar);
  TinyTensor<Type>& floatks(float k);
  TinyTensor<Type>& resize(const std::vector<int>& new_shape);

  TinyTensor<Type> ReluForward() const;
  TinyTensor<Type> ReluBackward(const TinyTensor<Type>& grad) const;
  TinyTensor<Type> SigmoidForward() const;
  TinyTensor<Type> SigmoidBackward(const TinyTensor<Type>& grad) const;

  bool on_gpu() const { return device == "gpu"; }

 private:
  void allocate();
  void release();
  // Elementwise op via the C-ABI (gpu) or a host loop (cpu); writes into *this.
  void apply(int op, const TinyTensor<Type>* a, const TinyTensor<Type>* b, double alpha, double beta,
             uint64_t seed);
};

template <typename T>
std::ostream& operator<<(std::ostream& os, const TinyTensor<T>& t);
