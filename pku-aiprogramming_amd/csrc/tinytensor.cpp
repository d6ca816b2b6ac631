// TinyTensor<T> implementation over the C-ABI.  Host-only C++ (built with
// g++); every device interaction goes through include/tt_attn.h.
//
// Method semantics follow the reference (Task3/Tinytensor/src/Tinytensor.cu):
// constructors :13-83, destructor :85-93, Size :95-102, operator= :104-127,
// +/- :129-171 (shape and device mismatch -> invalid_argument), [] :173-196
// (index range check), get_data :208-220, flatten :222-232, cpu/gpu
// :234-257, random :259-292, zeros/ones/negative/mults/floatks :294-354,
// resize :356-382 (keeps the leading min(old, new) elements), activations
// :384-485 (CPU-side gradient tensors are staged to the device), printing
// :487-517.
#include "tinytensor.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <random>
#include <sstream>
#include <stdexcept>
#include <type_traits>

namespace py = pybind11;

void tt_check(int rc, const char* what) {
  if (rc == TT_OK) return;
  std::string msg = std::string(what) + ": " + tt_last_error();
  if (rc == TT_ERR_ARG || rc == TT_ERR_UNSUPPORTED) throw std::invalid_argument(msg);
  throw std::runtime_error(msg);
}

static size_t shape_size(const std::vector<int>& shape) {
  size_t n = 1;
  for (int d : shape) {
    if (d < 0) throw std::invalid_argument("Negative dimension");
    n *= (size_t)d;
  }
  return n;
}

static void check_device(const std::string& dev) {
  if (dev != "cpu" && dev != "gpu") throw std::invalid_argument("Invalid device");
}

// n host values -> device storage, and back; synchronous.  bf16 converts in
// the library's staging pass; every other dtype stores its host type as is.
template <typename T>
static void upload(T* dev, const typename Dtype<T>::host* src, size_t n) {
  if constexpr (std::is_same<T, bf16>::value)
    tt_check(tt_upload_bf16_from_f32(dev, src, n), "TinyTensor upload");
  else
    tt_check(tt_memcpy_h2d(dev, src, n * sizeof(T)), "TinyTensor upload");
}
template <typename T>
static void download(typename Dtype<T>::host* dst, const T* dev, size_t n) {
  if constexpr (std::is_same<T, bf16>::value)
    tt_check(tt_download_bf16_to_f32(dst, dev, n), "TinyTensor download");
  else
    tt_check(tt_memcpy_d2h(dst, dev, n * sizeof(T)), "TinyTensor download");
}

template <typename T>
void TinyTensor<T>::allocate() {
  size = shape_size(shape);
  if (device == "cpu") {
    p_data = new T[size > 0 ? size : 1];
  } else {
    void* p = nullptr;
    tt_check(tt_malloc(&p, std::max<size_t>(size, 1) * sizeof(T)), "TinyTensor allocation");
    p_data = static_cast<T*>(p);
  }
}

template <typename T>
void TinyTensor<T>::release() {
  if (!p_data) return;
  if (device == "cpu")
    delete[] p_data;
  else
    tt_free(p_data);
  p_data = nullptr;
}

template <typename T>
TinyTensor<T>::TinyTensor(const std::vector<int>& shape_, const std::string& device_)
    : shape(shape_), device(device_) {
  check_device(device);
  allocate();
}

template <typename T>
TinyTensor<T>::TinyTensor(const std::vector<int>& shape_, const std::string& device_,
                          const std::vector<Host>& data)
    : shape(shape_), device(device_) {
  check_device(device);
  allocate();
  // Like the reference, copy min(size, data.size()) leading values; the rest
  // of the storage is zero here rather than uninitialised.
  if (device == "cpu") {
    for (size_t i = 0; i < size; ++i) p_data[i] = Dtype<T>::from_host(i < data.size() ? data[i] : Host(0));
  } else if (data.size() >= size) {
    upload(p_data, data.data(), size);
  } else {
    std::vector<Host> padded(size, Host(0));
    std::copy(data.begin(), data.end(), padded.begin());
    upload(p_data, padded.data(), size);
  }
}

template <typename T>
TinyTensor<T>::TinyTensor(const py::array_t<Host>& data, const std::string& device_) : device(device_) {
  check_device(device);
  // Force a C-contiguous view (the reference copies buffer.ptr raw, which is
  // wrong for non-contiguous inputs).
  py::array_t<Host, py::array::c_style | py::array::forcecast> a(data);
  py::buffer_info buf = a.request();
  for (auto dim : buf.shape) shape.push_back((int)dim);
  allocate();
  const Host* src = static_cast<const Host*>(buf.ptr);
  if (device == "cpu") {
    for (size_t i = 0; i < size; ++i) p_data[i] = Dtype<T>::from_host(src[i]);
  } else {
    upload(p_data, src, size);
  }
}

template <typename T>
TinyTensor<T>::TinyTensor(const TinyTensor<T>& other) : shape(other.shape), device(other.device) {
  allocate();
  if (device == "cpu")
    std::copy(other.p_data, other.p_data + size, p_data);
  else
    tt_check(tt_memcpy_d2d(p_data, other.p_data, size * sizeof(T)), "TinyTensor copy");
}

template <typename T>
TinyTensor<T>::~TinyTensor() {
  release();
}

template <typename T>
size_t TinyTensor<T>::Size() const {
  return shape_size(shape);
}

template <typename T>
TinyTensor<T>& TinyTensor<T>::operator=(const TinyTensor<T>& other) {
  if (this == &other) return *this;
  release();
  shape = other.shape;
  device = other.device;
  allocate();
  if (device == "cpu")
    std::copy(other.p_data, other.p_data + size, p_data);
  else
    tt_check(tt_memcpy_d2d(p_data, other.p_data, size * sizeof(T)), "TinyTensor assign");
  return *this;
}

template <typename T>
void TinyTensor<T>::apply(int op, const TinyTensor<T>* a, const TinyTensor<T>* b, double alpha, double beta,
                          uint64_t seed) {
  if (device == "gpu") {
    tt_check(tt_elementwise(op, Dtype<T>::code, p_data, a ? a->p_data : nullptr, b ? b->p_data : nullptr,
                            (int64_t)size, alpha, beta, seed, nullptr),
             "TinyTensor elementwise");
    return;
  }
  using H = Host;
  for (size_t i = 0; i < size; ++i) {
    H x = a ? Dtype<T>::to_host(a->p_data[i]) : H(0);
    H y = b ? Dtype<T>::to_host(b->p_data[i]) : H(0);
    H r = 0;
    switch (op) {
      case TT_EW_ADD: r = x + y; break;
      case TT_EW_SUB: r = x - y; break;
      case TT_EW_FILL: r = (H)alpha; break;
      case TT_EW_NEG: r = -x; break;
      case TT_EW_SCALE: r = (H)(x * (H)alpha); break;
      case TT_EW_RELU: r = x > 0 ? x : H(0); break;
      case TT_EW_RELU_BWD: r = x > 0 ? y : H(0); break;
      case TT_EW_SIGMOID: r = (H)(1.0 / (1.0 + std::exp(-(double)x))); break;
      case TT_EW_SIGMOID_BWD: {
        double s = 1.0 / (1.0 + std::exp(-(double)x));
        r = (H)(s * (1.0 - s) * (double)y);
      } break;
      default: throw std::invalid_argument("bad elementwise op");
    }
    p_data[i] = Dtype<T>::from_host(r);
  }
}

template <typename T>
TinyTensor<T> TinyTensor<T>::operator+(const TinyTensor<T>& other) const {
  if (shape != other.shape) throw std::invalid_argument("Shape mismatch");
  if (device != other.device) throw std::invalid_argument("Device mismatch");
  TinyTensor<T> result{shape, device};
  result.apply(TT_EW_ADD, this, &other, 0, 0, 0);
  return result;
}

template <typename T>
TinyTensor<T> TinyTensor<T>::operator-(const TinyTensor<T>& other) const {
  if (shape != other.shape) throw std::invalid_argument("Shape mismatch");
  if (device != other.device) throw std::invalid_argument("Device mismatch");
  TinyTensor<T> result{shape, device};
  result.apply(TT_EW_SUB, this, &other, 0, 0, 0);
  return result;
}

template <typename T>
TinyTensor<T> TinyTensor<T>::operator[](int k) const {
  if (shape.empty() || k < 0 || k >= shape[0]) throw std::invalid_argument("Index out of range");
  std::vector<int> new_shape(shape.begin() + 1, shape.end());
  if (new_shape.empty()) new_shape.push_back(1);
  const size_t n = shape_size(std::vector<int>(shape.begin() + 1, shape.end()));
  TinyTensor<T> result{new_shape, device};
  if (device == "cpu")
    std::copy(p_data + (size_t)k * n, p_data + (size_t)(k + 1) * n, result.p_data);
  else
    tt_check(tt_memcpy_d2d(result.p_data, p_data + (size_t)k * n, n * sizeof(T)), "TinyTensor slice");
  return result;
}

template <typename T>
std::vector<int> TinyTensor<T>::get_shape() const {
  return shape;
}

template <typename T>
std::string TinyTensor<T>::get_device() const {
  return device;
}

template <typename T>
std::vector<typename TinyTensor<T>::Host> TinyTensor<T>::get_data() const {
  std::vector<Host> out(size);
  if (device == "cpu")
    for (size_t i = 0; i < size; ++i) out[i] = Dtype<T>::to_host(p_data[i]);
  else
    download(out.data(), p_data, size);
  return out;
}

template <typename T>
py::array_t<typename TinyTensor<T>::Host> TinyTensor<T>::numpy() const {
  std::vector<py::ssize_t> dims(shape.begin(), shape.end());
  py::array_t<Host> out(dims);
  Host* dst = out.mutable_data();
  if (device == "cpu")
    for (size_t i = 0; i < size; ++i) dst[i] = Dtype<T>::to_host(p_data[i]);
  else
    download(dst, p_data, size);
  return out;
}

template <typename T>
TinyTensor<T> TinyTensor<T>::flatten() const {
  // [N, ...] -> [N, rest]: the batch is the product of all but the last three
  // axes (reference :222-232); rank < 3 keeps the whole tensor as one row.
  int batch = 1;
  for (size_t i = 0; i + 3 < shape.size(); ++i) batch *= shape[i];
  TinyTensor<T> result(*this);
  const int rest = batch > 0 ? (int)(size / (size_t)batch) : 0;
  result.resize(std::vector<int>{batch, rest});
  return result;
}

template <typename T>
TinyTensor<T>& TinyTensor<T>::cpu() {
  if (device == "gpu") {
    T* host = new T[size > 0 ? size : 1];
    int rc = tt_memcpy_d2h(host, p_data, size * sizeof(T));
    if (rc != TT_OK) {
      delete[] host;
      tt_check(rc, "TinyTensor.cpu");
    }
    tt_free(p_data);
    p_data = host;
    device = "cpu";
  }
  return *this;
}

template <typename T>
TinyTensor<T>& TinyTensor<T>::gpu() {
  if (device == "cpu") {
    void* d = nullptr;
    tt_check(tt_malloc(&d, std::max<size_t>(size, 1) * sizeof(T)), "TinyTensor.gpu");
    int rc = tt_memcpy_h2d(d, p_data, size * sizeof(T));
    if (rc != TT_OK) {
      tt_free(d);
      tt_check(rc, "TinyTensor.gpu");
    }
    delete[] p_data;
    p_data = static_cast<T*>(d);
    device = "gpu";
  }
  return *this;
}

template <typename T>
TinyTensor<T>& TinyTensor<T>::random(Host a, Host b) {
  // Unseeded, like the reference (std::random_device on the CPU, a clock seed
  // on the GPU): U[a, b) for floating types, [a, b] for int.
  std::random_device rd;
  const uint64_t seed = (uint64_t(rd()) << 32) ^ rd();
  if (device == "gpu") {
    apply(TT_EW_UNIFORM, nullptr, nullptr, (double)a, (double)b, seed);
  } else {
    std::mt19937_64 gen(seed);
    if constexpr (std::is_integral<Host>::value) {
      std::uniform_int_distribution<Host> dist(a, b);
      for (size_t i = 0; i < size; ++i) p_data[i] = Dtype<T>::from_host(dist(gen));
    } else {
      std::uniform_real_distribution<Host> dist(a, b);
      for (size_t i = 0; i < size; ++i) p_data[i] = Dtype<T>::from_host(dist(gen));
    }
  }
  return *this;
}

template <typename T>
TinyTensor<T>& TinyTensor<T>::zeros() {
  if (device == "cpu")
    std::fill(p_data, p_data + size, Dtype<T>::from_host(Host(0)));
  else
    tt_check(tt_memset(p_data, 0, size * sizeof(T)), "TinyTensor.zeros");
  return *this;
}

template <typename T>
TinyTensor<T>& TinyTensor<T>::ones() {
  apply(TT_EW_FILL, nullptr, nullptr, 1.0, 0, 0);
  return *this;
}

template <typename T>
TinyTensor<T>& TinyTensor<T>::negative() {
  apply(TT_EW_NEG, this, nullptr, 0, 0, 0);
  return *this;
}

template <typename T>
TinyTensor<T>& TinyTensor<T>::mults(Host scalar) {
  apply(TT_EW_SCALE, this, nullptr, (double)scalar, 0, 0);
  return *this;
}

template <typename T>
TinyTensor<T>& TinyTensor<T>::floatks(float k) {
  apply(TT_EW_FILL, nullptr, nullptr, (double)k, 0, 0);
  return *this;
}

template <typename T>
TinyTensor<T>& TinyTensor<T>::resize(const std::vector<int>& new_shape) {
  const size_t new_size = shape_size(new_shape);
  const size_t old_size = size;
  shape = new_shape;
  size = new_size;
  if (new_size == old_size) return *this;
  const size_t keep = std::min(old_size, new_size);
  if (device == "cpu") {
    T* nd = new T[new_size > 0 ? new_size : 1];
    std::copy(p_data, p_data + keep, nd);
    delete[] p_data;
    p_data = nd;
  } else {
    void* nd = nullptr;
    tt_check(tt_malloc(&nd, std::max<size_t>(new_size, 1) * sizeof(T)), "TinyTensor.resize");
    int rc = tt_memcpy_d2d(nd, p_data, keep * sizeof(T));
    if (rc != TT_OK) {
      tt_free(nd);
      tt_check(rc, "TinyTensor.resize");
    }
    tt_free(p_data);
    p_data = static_cast<T*>(nd);
  }
  return *this;
}

template <typename T>
TinyTensor<T> TinyTensor<T>::ReluForward() const {
  TinyTensor<T> result{*this};
  result.apply(TT_EW_RELU, &result, nullptr, 0, 0, 0);
  return result;
}

template <typename T>
TinyTensor<T> TinyTensor<T>::ReluBackward(const TinyTensor<T>& grad) const {
  if (grad.size != size) throw std::invalid_argument("Shape mismatch");
  TinyTensor<T> result{*this};
  TinyTensor<T> g{grad};
  if (device == "gpu") g.gpu(); else g.cpu();
  result.apply(TT_EW_RELU_BWD, &result, &g, 0, 0, 0);
  return result;
}

template <typename T>
TinyTensor<T> TinyTensor<T>::SigmoidForward() const {
  TinyTensor<T> result{*this};
  result.apply(TT_EW_SIGMOID, &result, nullptr, 0, 0, 0);
  return result;
}

template <typename T>
TinyTensor<T> TinyTensor<T>::SigmoidBackward(const TinyTensor<T>& grad) const {
  if (grad.size != size) throw std::invalid_argument("Shape mismatch");
  TinyTensor<T> result{*this};
  TinyTensor<T> g{grad};
  if (device == "gpu") g.gpu(); else g.cpu();
  result.apply(TT_EW_SIGMOID_BWD, &result, &g, 0, 0, 0);
  return result;
}

template <typename T>
std::ostream& operator<<(std::ostream& os, const TinyTensor<T>& t) {
  os << "TinyTensor<" << Dtype<T>::name << ">\n";
  os << "Device: " << t.device << "\nShape: [";
  for (size_t i = 0; i < t.shape.size(); ++i) {
    os << t.shape[i];
    if (i + 1 < t.shape.size()) os << ", ";
  }
  os << "]\n";
  const auto data = t.get_data();
  const size_t row = t.shape.empty() || t.shape.back() == 0 ? 1 : (size_t)t.shape.back();
  for (size_t i = 0; i < data.size(); ++i) {
    os << data[i] << " ";
    if ((i + 1) % row == 0) os << "\n";
  }
  return os;
}

template class TinyTensor<int>;
template class TinyTensor<float>;
template class TinyTensor<double>;
template class TinyTensor<bf16>;
template std::ostream& operator<<(std::ostream&, const TinyTensor<int>&);
template std::ostream& operator<<(std::ostream&, const TinyTensor<float>&);
template std::ostream& operator<<(std::ostream&, const TinyTensor<double>&);
template std::ostream& operator<<(std::ostream&, const TinyTensor<bf16>&);
