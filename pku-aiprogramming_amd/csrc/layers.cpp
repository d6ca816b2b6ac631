// Attention, softmax and fully connected layer functions: shape checks, output sizing, then the C-ABI calls.
#include "layers.h"

#include <initializer_list>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <utility>

namespace {

void need_gpu(const std::string& fn, const std::string& name, const std::string& dev) {
  if (dev != "gpu") throw std::invalid_argument(fn + ": " + name + " must be on device \"gpu\"");
}

struct Dims {
  int B, H, L, d;
};

template <typename T>
Dims dims4(const std::string& fn, const std::string& name, const TinyTensor<T>& t) {
  if (t.shape.size() != 4)
    throw std::invalid_argument(fn + ": " + name + " must have rank 4 [B, H, L, d]");
  return Dims{t.shape[0], t.shape[1], t.shape[2], t.shape[3]};
}

template <typename T>
void check_qkv(const std::string& fn, const TinyTensor<T>& q, const TinyTensor<T>& k, const TinyTensor<T>& v,
               Dims& dq, Dims& dk) {
  need_gpu(fn, "q", q.device);
  need_gpu(fn, "k", k.device);
  need_gpu(fn, "v", v.device);
  dq = dims4(fn, "q", q);
  dk = dims4(fn, "k", k);
  Dims dv = dims4(fn, "v", v);
  if (dq.B != dk.B || dq.H != dk.H || dq.d != dk.d)
    throw std::invalid_argument(fn + ": q and k disagree on B, H or d");
  if (dv.B != dk.B || dv.H != dk.H || dv.L != dk.L || dv.d != dk.d)
    throw std::invalid_argument(fn + ": k and v must have the same shape");
}

// Outputs must not share storage with an input or with each other: the
// kernels read the inputs while they write the outputs, and an output's
// resize may free the storage it held.  (Distinct tensors never share
// storage: copies are deep, so equal data pointers mean the same tensor.)
using Named = std::pair<const void*, const char*>;
void no_alias(const std::string& fn, std::initializer_list<Named> inputs, std::initializer_list<Named> outputs) {
  for (auto o = outputs.begin(); o != outputs.end(); ++o) {
    if (!o->first) continue;
    for (const Named& i : inputs)
      if (i.first == o->first)
        throw std::invalid_argument(fn + ": output " + o->second + " is the same tensor as input " + i.second);
    for (auto o2 = outputs.begin(); o2 != o; ++o2)
      if (o2->first == o->first)
        throw std::invalid_argument(fn + ": outputs " + o2->second + " and " + o->second + " are the same tensor");
  }
}

}  // namespace

template <typename T>
void AttentionForward(const TinyTensor<T>& q, const TinyTensor<T>& k, const TinyTensor<T>& v,
                      TinyTensor<T>& out, TinyTensor<float>& lse, float scale, bool causal) {
  const std::string fn = "AttentionForward";
  Dims dq, dk;
  check_qkv(fn, q, k, v, dq, dk);
  need_gpu(fn, "out", out.device);
  need_gpu(fn, "lse", lse.device);
  no_alias(fn, {{q.p_data, "q"}, {k.p_data, "k"}, {v.p_data, "v"}}, {{out.p_data, "out"}, {lse.p_data, "lse"}});
  out.resize(q.shape);
  lse.resize(std::vector<int>{dq.B, dq.H, dq.L});
  int rc;
  if constexpr (std::is_same<T, float>::value)
    rc = tt_attn_fwd_f32(q.p_data, k.p_data, v.p_data, out.p_data, lse.p_data, dq.B, dq.H, dq.L, dk.L, dq.d,
                         scale, causal ? 1 : 0, nullptr);
  else
    rc = tt_attn_fwd_bf16(reinterpret_cast<const uint16_t*>(q.p_data), reinterpret_cast<const uint16_t*>(k.p_data),
                          reinterpret_cast<const uint16_t*>(v.p_data), reinterpret_cast<uint16_t*>(out.p_data),
                          lse.p_data, dq.B, dq.H, dq.L, dk.L, dq.d, scale, causal ? 1 : 0, nullptr);
  tt_check(rc, fn.c_str());
  tt_check(tt_sync(), fn.c_str());
}

template <typename T>
void AttentionBackward(const TinyTensor<T>& q, const TinyTensor<T>& k, const TinyTensor<T>& v,
                       const TinyTensor<T>& out, const TinyTensor<float>& lse,
                       const TinyTensor<T>& grad_out, TinyTensor<T>& grad_q, TinyTensor<T>& grad_k,
                       TinyTensor<T>& grad_v, float scale, bool causal) {
  const std::string fn = "AttentionBackward";
  Dims dq, dk;
  check_qkv(fn, q, k, v, dq, dk);
  need_gpu(fn, "out", out.device);
  need_gpu(fn, "lse", lse.device);
  need_gpu(fn, "grad_out", grad_out.device);
  need_gpu(fn, "grad_q", grad_q.device);
  need_gpu(fn, "grad_k", grad_k.device);
  need_gpu(fn, "grad_v", grad_v.device);
  if (out.shape != q.shape) throw std::invalid_argument(fn + ": out must have the shape of q");
  if (grad_out.shape != q.shape) throw std::invalid_argument(fn + ": grad_out must have the shape of q");
  if (lse.shape != std::vector<int>{dq.B, dq.H, dq.L})
    throw std::invalid_argument(fn + ": lse must have shape [B, H, Lq]");
  no_alias(fn,
           {{q.p_data, "q"}, {k.p_data, "k"}, {v.p_data, "v"}, {out.p_data, "out"}, {lse.p_data, "lse"},
            {grad_out.p_data, "grad_out"}},
           {{grad_q.p_data, "grad_q"}, {grad_k.p_data, "grad_k"}, {grad_v.p_data, "grad_v"}});
  grad_q.resize(q.shape);
  grad_k.resize(k.shape);
  grad_v.resize(v.shape);
  int rc;
  if constexpr (std::is_same<T, float>::value)
    rc = tt_attn_bwd_f32(q.p_data, k.p_data, v.p_data, out.p_data, lse.p_data, grad_out.p_data, grad_q.p_data,
                         grad_k.p_data, grad_v.p_data, dq.B, dq.H, dq.L, dk.L, dq.d, scale, causal ? 1 : 0,
                         nullptr);
  else
    rc = tt_attn_bwd_bf16(
        reinterpret_cast<const uint16_t*>(q.p_data), reinterpret_cast<const uint16_t*>(k.p_data),
        reinterpret_cast<const uint16_t*>(v.p_data), reinterpret_cast<const uint16_t*>(out.p_data), lse.p_data,
        reinterpret_cast<const uint16_t*>(grad_out.p_data), reinterpret_cast<uint16_t*>(grad_q.p_data),
        reinterpret_cast<uint16_t*>(grad_k.p_data), reinterpret_cast<uint16_t*>(grad_v.p_data), dq.B, dq.H, dq.L,
        dk.L, dq.d, scale, causal ? 1 : 0, nullptr);
  tt_check(rc, fn.c_str());
  tt_check(tt_sync(), fn.c_str());
}

template <typename T>
void AttentionDecode(const TinyTensor<T>& q, const TinyTensor<T>& k_cache, const TinyTensor<T>& v_cache,
                     TinyTensor<T>& out, float scale) {
  const std::string fn = "AttentionDecode";
  Dims dq, dk;
  check_qkv(fn, q, k_cache, v_cache, dq, dk);
  need_gpu(fn, "out", out.device);
  if (dq.L != 1) throw std::invalid_argument(fn + ": q must have Lq == 1");
  no_alias(fn, {{q.p_data, "q"}, {k_cache.p_data, "k_cache"}, {v_cache.p_data, "v_cache"}}, {{out.p_data, "out"}});
  out.resize(q.shape);
  int rc;
  if constexpr (std::is_same<T, float>::value)
    rc = tt_attn_decode_f32(q.p_data, k_cache.p_data, v_cache.p_data, out.p_data, nullptr, dq.B, dq.H, dk.L,
                            dq.d, scale, nullptr);
  else
    rc = tt_attn_decode_bf16(reinterpret_cast<const uint16_t*>(q.p_data),
                             reinterpret_cast<const uint16_t*>(k_cache.p_data),
                             reinterpret_cast<const uint16_t*>(v_cache.p_data),
                             reinterpret_cast<uint16_t*>(out.p_data), nullptr, dq.B, dq.H, dk.L, dq.d, scale,
                             nullptr);
  tt_check(rc, fn.c_str());
  tt_check(tt_sync(), fn.c_str());
}

template <typename T>
void SoftmaxForward(const TinyTensor<T>& input, TinyTensor<T>& output) {
  static_assert(std::is_same<T, float>::value, "SoftmaxForward is float only, as in the reference");
  const std::string fn = "SoftmaxForward";
  need_gpu(fn, "input", input.device);
  if (input.shape.empty()) throw std::invalid_argument(fn + ": input must have rank >= 1");
  int64_t rows = 1;
  for (size_t i = 0; i + 1 < input.shape.size(); ++i) rows *= input.shape[i];
  const int64_t cols = input.shape.back();
  if (&output != &input) {
    if (output.device != "gpu") output.gpu();
    output.resize(input.shape);
  }
  tt_check(tt_softmax_rows_f32(input.p_data, output.p_data, rows, cols, nullptr), fn.c_str());
  tt_check(tt_sync(), fn.c_str());
}

namespace {

// C = alpha op(A) op(B) + beta C on the library GEMM (row-major, tt_gemm_*).
template <typename T>
void gemm(const char* fn, bool ta, bool tb, int64_t m, int64_t n, int64_t k, float alpha, const T* A, const T* B,
          float beta, T* C) {
  int rc;
  if constexpr (std::is_same<T, float>::value)
    rc = tt_gemm_f32(ta ? 1 : 0, tb ? 1 : 0, m, n, k, alpha, A, B, beta, C, nullptr);
  else
    rc = tt_gemm_bf16(ta ? 1 : 0, tb ? 1 : 0, m, n, k, alpha, reinterpret_cast<const uint16_t*>(A),
                      reinterpret_cast<const uint16_t*>(B), beta, reinterpret_cast<uint16_t*>(C), nullptr);
  tt_check(rc, fn);
}

struct FcDims {
  int64_t batch, fin, fout;
  bool scalar_bias;
};

// The reference's reading of the shapes (Layers.cu:16-24, 28): every axis of
// input but the last is a batch axis, weight is [fin, fout], a bias of shape
// [1] is one value for every output, any other bias is the [fout] row.
template <typename T>
FcDims fc_dims(const std::string& fn, const TinyTensor<T>& input, const TinyTensor<T>& weight,
               const TinyTensor<T>& bias) {
  need_gpu(fn, "input", input.device);
  need_gpu(fn, "weight", weight.device);
  need_gpu(fn, "bias", bias.device);
  if (input.shape.empty()) throw std::invalid_argument(fn + ": input must have rank >= 1");
  if (weight.shape.size() != 2) throw std::invalid_argument(fn + ": weight must have rank 2 [fin, fout]");
  FcDims f;
  f.batch = 1;
  for (size_t i = 0; i + 1 < input.shape.size(); ++i) f.batch *= input.shape[i];
  f.fin = input.shape.back();
  f.fout = weight.shape[1];
  if (weight.shape[0] != f.fin)
    throw std::invalid_argument(fn + ": weight rows (" + std::to_string(weight.shape[0]) +
                                ") must equal the input's last axis (" + std::to_string(f.fin) + ")");
  f.scalar_bias = bias.shape.size() == 1 && bias.shape[0] == 1;
  if (!f.scalar_bias && (int64_t)bias.size != f.fout)
    throw std::invalid_argument(fn + ": bias must hold fout (" + std::to_string(f.fout) + ") values or be [1]");
  return f;
}

}  // namespace

template <typename T>
void FcForward(const TinyTensor<T>& input, TinyTensor<T>& output, const TinyTensor<T>& weight,
               const TinyTensor<T>& bias) {
  const std::string fn = "FcForward";
  const FcDims f = fc_dims(fn, input, weight, bias);
  need_gpu(fn, "output", output.device);
  no_alias(fn, {{input.p_data, "input"}, {weight.p_data, "weight"}, {bias.p_data, "bias"}},
           {{output.p_data, "output"}});
  std::vector<int> oshape(input.shape.begin(), input.shape.end() - 1);
  oshape.push_back((int)f.fout);
  output.resize(oshape);
  if (f.batch == 0 || f.fout == 0) return;
  gemm<T>(fn.c_str(), false, false, f.batch, f.fout, f.fin, 1.f, input.p_data, weight.p_data, 0.f, output.p_data);
  TinyTensor<T> ones(std::vector<int>{(int)f.batch, 1}, "gpu");
  ones.ones();
  if (f.scalar_bias) {
    TinyTensor<T> row(std::vector<int>{1, (int)f.fout}, "gpu");
    row.floatks((float)bias.get_data()[0]);
    gemm<T>(fn.c_str(), false, false, f.batch, f.fout, 1, 1.f, ones.p_data, row.p_data, 1.f, output.p_data);
    tt_check(tt_sync(), fn.c_str());
  } else {
    gemm<T>(fn.c_str(), false, false, f.batch, f.fout, 1, 1.f, ones.p_data, bias.p_data, 1.f, output.p_data);
    tt_check(tt_sync(), fn.c_str());
  }
}

template <typename T>
void FcBackward(const TinyTensor<T>& input, const TinyTensor<T>& output, const TinyTensor<T>& weight,
                const TinyTensor<T>& bias, TinyTensor<T>& grad_input, const TinyTensor<T>& grad_output,
                TinyTensor<T>& grad_weight, TinyTensor<T>& grad_bias) {
  (void)output;
  const std::string fn = "FcBackward";
  const FcDims f = fc_dims(fn, input, weight, bias);
  need_gpu(fn, "grad_output", grad_output.device);
  need_gpu(fn, "grad_input", grad_input.device);
  need_gpu(fn, "grad_weight", grad_weight.device);
  need_gpu(fn, "grad_bias", grad_bias.device);
  if ((int64_t)grad_output.size != f.batch * f.fout || grad_output.shape.empty() ||
      grad_output.shape.back() != f.fout)
    throw std::invalid_argument(fn + ": grad_output must be [.., fout] with the input's batch axes");
  no_alias(fn,
           {{input.p_data, "input"}, {weight.p_data, "weight"}, {bias.p_data, "bias"},
            {grad_output.p_data, "grad_output"}},
           {{grad_input.p_data, "grad_input"}, {grad_weight.p_data, "grad_weight"}, {grad_bias.p_data, "grad_bias"}});
  grad_input.resize(input.shape);
  grad_weight.resize(weight.shape);
  grad_bias.resize(bias.shape);
  if (f.batch == 0) {  // no rows: every gradient is a sum over nothing
    grad_weight.zeros();
    grad_bias.zeros();
    tt_check(tt_sync(), fn.c_str());
    return;
  }
  if (f.fout == 0) {
    grad_input.zeros();
    grad_bias.zeros();
    tt_check(tt_sync(), fn.c_str());
    return;
  }
  gemm<T>(fn.c_str(), false, true, f.batch, f.fin, f.fout, 1.f, grad_output.p_data, weight.p_data, 0.f,
          grad_input.p_data);
  gemm<T>(fn.c_str(), true, false, f.fin, f.fout, f.batch, 1.f, input.p_data, grad_output.p_data, 0.f,
          grad_weight.p_data);
  TinyTensor<T> ones(std::vector<int>{1, (int)f.batch}, "gpu");
  ones.ones();
  if (f.scalar_bias) {
    TinyTensor<T> row(std::vector<int>{1, (int)f.fout}, "gpu");
    gemm<T>(fn.c_str(), false, false, 1, f.fout, f.batch, 1.f, ones.p_data, grad_output.p_data, 0.f, row.p_data);
    TinyTensor<T> col(std::vector<int>{(int)f.fout, 1}, "gpu");
    col.ones();
    gemm<T>(fn.c_str(), false, false, 1, 1, f.fout, 1.f, row.p_data, col.p_data, 0.f, grad_bias.p_data);
    tt_check(tt_sync(), fn.c_str());
  } else {
    gemm<T>(fn.c_str(), false, false, 1, f.fout, f.batch, 1.f, ones.p_data, grad_output.p_data, 0.f,
            grad_bias.p_data);
    tt_check(tt_sync(), fn.c_str());
  }
}

namespace {

struct ConvShape {
  int64_t batch;
  int C, H, W;
};

// The reference's reading of an image tensor (Layers.cu:91-97): the last three
// axes are C, H, W, the others batch axes.
ConvShape conv_shape(const std::string& fn, const std::string& name, const std::vector<int>& shape) {
  if (shape.size() < 3) throw std::invalid_argument(fn + ": " + name + " must have rank >= 3 [.., C, H, W]");
  ConvShape c{1, shape[shape.size() - 3], shape[shape.size() - 2], shape.back()};
  for (size_t i = 0; i + 3 < shape.size(); ++i) c.batch *= shape[i];
  return c;
}

// Output extent of one axis; throws where the C-ABI would refuse the shape.
int conv_out(const std::string& fn, int in, int k, int pad, int stride) {
  if (k < 1 || pad < 0 || stride < 1)
    throw std::invalid_argument(fn + ": kernel sizes >= 1, pads >= 0 and strides >= 1 required");
  if ((int64_t)in + 2 * (int64_t)pad < k) throw std::invalid_argument(fn + ": the kernel is larger than the padded image");
  return (int)((in + 2 * (int64_t)pad - k) / stride + 1);
}

template <typename T>
int dtype_code() {
  return std::is_same<T, float>::value ? TT_F32 : TT_BF16;
}

template <typename T>
void im2col_call(const std::string& fn, const T* im, T* col, const ConvShape& s, int kh, int kw, int ph, int pw,
                 int sh, int sw) {
  tt_check(tt_im2col(dtype_code<T>(), im, col, s.batch, s.C, s.H, s.W, kh, kw, ph, pw, sh, sw, nullptr),
           fn.c_str());
}

template <typename T>
void col2im_call(const std::string& fn, const T* col, T* im, const ConvShape& s, int kh, int kw, int ph, int pw,
                 int sh, int sw) {
  tt_check(tt_col2im(dtype_code<T>(), col, im, s.batch, s.C, s.H, s.W, kh, kw, ph, pw, sh, sw, nullptr),
           fn.c_str());
}

}  // namespace

template <typename T>
void Im2col(const TinyTensor<T>& im_tensor, TinyTensor<T>& col_tensor, const std::vector<int>& kernel_shape,
            int pad_h, int pad_w, int stride_h, int stride_w) {
  const std::string fn = "im2col";
  need_gpu(fn, "im_tensor", im_tensor.device);
  need_gpu(fn, "col_tensor", col_tensor.device);
  if (kernel_shape.size() < 2) throw std::invalid_argument(fn + ": kernel_shape must end with [kh, kw]");
  const ConvShape s = conv_shape(fn, "im_tensor", im_tensor.shape);
  const int kh = kernel_shape[kernel_shape.size() - 2], kw = kernel_shape.back();
  const int oh = conv_out(fn, s.H, kh, pad_h, stride_h), ow = conv_out(fn, s.W, kw, pad_w, stride_w);
  no_alias(fn, {{im_tensor.p_data, "im_tensor"}}, {{col_tensor.p_data, "col_tensor"}});
  const int P = oh * ow, K = s.C * kh * kw;
  if (im_tensor.shape.size() == 3)
    col_tensor.resize(std::vector<int>{P, K});
  else
    col_tensor.resize(std::vector<int>{(int)s.batch, P, K});
  im2col_call(fn, im_tensor.p_data, col_tensor.p_data, s, kh, kw, pad_h, pad_w, stride_h, stride_w);
  tt_check(tt_sync(), fn.c_str());
}

template <typename T>
void Col2im(const TinyTensor<T>& col_tensor, TinyTensor<T>& im_tensor, const std::vector<int>& kernel_shape,
            const std::vector<int>& im_shape, int pad_h, int pad_w, int stride_h, int stride_w) {
  const std::string fn = "col2im";
  need_gpu(fn, "col_tensor", col_tensor.device);
  need_gpu(fn, "im_tensor", im_tensor.device);
  if (kernel_shape.size() < 2) throw std::invalid_argument(fn + ": kernel_shape must end with [kh, kw]");
  const ConvShape s = conv_shape(fn, "im_shape", im_shape);
  const int kh = kernel_shape[kernel_shape.size() - 2], kw = kernel_shape.back();
  const int oh = conv_out(fn, s.H, kh, pad_h, stride_h), ow = conv_out(fn, s.W, kw, pad_w, stride_w);
  if ((int64_t)col_tensor.size != s.batch * oh * ow * (int64_t)s.C * kh * kw)
    throw std::invalid_argument(fn + ": col_tensor must hold batch x OH*OW x C*kh*kw values");
  no_alias(fn, {{col_tensor.p_data, "col_tensor"}}, {{im_tensor.p_data, "im_tensor"}});
  if (im_shape.size() == 3)
    im_tensor.resize(std::vector<int>{s.C, s.H, s.W});
  else
    im_tensor.resize(std::vector<int>{(int)s.batch, s.C, s.H, s.W});
  col2im_call(fn, col_tensor.p_data, im_tensor.p_data, s, kh, kw, pad_h, pad_w, stride_h, stride_w);
  tt_check(tt_sync(), fn.c_str());
}

namespace {

struct ConvDims {
  ConvShape in;
  int cout, kh, kw, oh, ow;
  int64_t P() const { return (int64_t)oh * ow; }
  int64_t K() const { return (int64_t)in.C * kh * kw; }
};

template <typename T>
ConvDims conv_dims(const std::string& fn, const TinyTensor<T>& input, const TinyTensor<T>& weight, int ph, int pw,
                   int sh, int sw) {
  need_gpu(fn, "input", input.device);
  need_gpu(fn, "weight", weight.device);
  ConvDims d;
  d.in = conv_shape(fn, "input", input.shape);
  if (weight.shape.size() != 4) throw std::invalid_argument(fn + ": weight must have rank 4 [Cout, Cin, kh, kw]");
  if (weight.shape[1] != d.in.C)
    throw std::invalid_argument(fn + ": weight's Cin (" + std::to_string(weight.shape[1]) +
                                ") must equal the input's channels (" + std::to_string(d.in.C) + ")");
  d.cout = weight.shape[0];
  d.kh = weight.shape[2];
  d.kw = weight.shape[3];
  d.oh = conv_out(fn, d.in.H, d.kh, ph, sh);
  d.ow = conv_out(fn, d.in.W, d.kw, pw, sw);
  return d;
}

}  // namespace

template <typename T>
void ConvForward(const TinyTensor<T>& input, TinyTensor<T>& output, const TinyTensor<T>& weight, int pad_h,
                 int pad_w, int stride_h, int stride_w) {
  const std::string fn = "ConvForward";
  const ConvDims d = conv_dims(fn, input, weight, pad_h, pad_w, stride_h, stride_w);
  need_gpu(fn, "output", output.device);
  no_alias(fn, {{input.p_data, "input"}, {weight.p_data, "weight"}}, {{output.p_data, "output"}});
  std::vector<int> oshape(input.shape.begin(), input.shape.end() - 3);
  oshape.insert(oshape.end(), {d.cout, d.oh, d.ow});
  output.resize(oshape);
  if (d.in.batch == 0 || d.cout == 0) return;
  const int64_t P = d.P(), K = d.K();
  TinyTensor<T> col(std::vector<int>{(int)d.in.batch, (int)P, (int)K}, "gpu");
  im2col_call(fn, input.p_data, col.p_data, d.in, d.kh, d.kw, pad_h, pad_w, stride_h, stride_w);
  for (int64_t n = 0; n < d.in.batch; ++n)
    gemm<T>(fn.c_str(), false, true, d.cout, P, K, 1.f, weight.p_data, col.p_data + n * P * K, 0.f,
            output.p_data + n * d.cout * P);
  tt_check(tt_sync(), fn.c_str());
}

template <typename T>
void ConvBackward(const TinyTensor<T>& input, const TinyTensor<T>& output, const TinyTensor<T>& weight,
                  TinyTensor<T>& grad_input, const TinyTensor<T>& grad_output, TinyTensor<T>& grad_weight,
                  int pad_h, int pad_w, int stride_h, int stride_w) {
  (void)output;
  const std::string fn = "ConvBackward";
  const ConvDims d = conv_dims(fn, input, weight, pad_h, pad_w, stride_h, stride_w);
  need_gpu(fn, "grad_output", grad_output.device);
  need_gpu(fn, "grad_input", grad_input.device);
  need_gpu(fn, "grad_weight", grad_weight.device);
  const int64_t P = d.P(), K = d.K();
  if ((int64_t)grad_output.size != d.in.batch * d.cout * P)
    throw std::invalid_argument(fn + ": grad_output must be [.., Cout, OH, OW] with the input's batch axes");
  no_alias(fn, {{input.p_data, "input"}, {weight.p_data, "weight"}, {grad_output.p_data, "grad_output"}},
           {{grad_input.p_data, "grad_input"}, {grad_weight.p_data, "grad_weight"}});
  grad_input.resize(input.shape);
  grad_weight.resize(weight.shape);
  if (d.in.batch == 0 || d.cout == 0) {  // sums over nothing
    grad_input.zeros();
    grad_weight.zeros();
    tt_check(tt_sync(), fn.c_str());
    return;
  }
  TinyTensor<T> col(std::vector<int>{(int)d.in.batch, (int)P, (int)K}, "gpu");
  im2col_call(fn, input.p_data, col.p_data, d.in, d.kh, d.kw, pad_h, pad_w, stride_h, stride_w);
  TinyTensor<T> grad_col(std::vector<int>{(int)d.in.batch, (int)P, (int)K}, "gpu");
  for (int64_t n = 0; n < d.in.batch; ++n) {
    const T* go = grad_output.p_data + n * d.cout * P;
    gemm<T>(fn.c_str(), false, false, d.cout, K, P, 1.f, go, col.p_data + n * P * K, n == 0 ? 0.f : 1.f,
            grad_weight.p_data);
    gemm<T>(fn.c_str(), true, false, P, K, d.cout, 1.f, go, weight.p_data, 0.f, grad_col.p_data + n * P * K);
  }
  col2im_call(fn, grad_col.p_data, grad_input.p_data, d.in, d.kh, d.kw, pad_h, pad_w, stride_h, stride_w);
  tt_check(tt_sync(), fn.c_str());
}

namespace {

// rows x classes of a softmax output, and its labels' count checked
template <typename T>
std::pair<int64_t, int64_t> ce_dims(const std::string& fn, const TinyTensor<T>& p, const TinyTensor<int>& labels) {
  if (p.shape.empty()) throw std::invalid_argument(fn + ": the softmax output must have rank >= 1");
  int64_t rows = 1;
  for (size_t i = 0; i + 1 < p.shape.size(); ++i) rows *= p.shape[i];
  if ((int64_t)labels.size != rows)
    throw std::invalid_argument(fn + ": labels must hold one class per row (" + std::to_string(rows) + ")");
  return {rows, (int64_t)p.shape.back()};
}

}  // namespace

template <typename T>
float SoftmaxLoss(const TinyTensor<T>& softmax_output, const TinyTensor<int>& labels) {
  static_assert(std::is_same<T, float>::value, "SoftmaxLoss is float only, as in the reference");
  const std::string fn = "SoftmaxLoss";
  const auto [rows, cols] = ce_dims(fn, softmax_output, labels);
  if (rows == 0) return 0.f;
  const std::vector<float> p = softmax_output.get_data();
  const std::vector<int> lab = labels.get_data();
  int64_t wrong = 0;
  for (int64_t i = 0; i < rows; ++i) {
    int64_t best = 0;
    for (int64_t j = 1; j < cols; ++j)
      if (p[i * cols + j] > p[i * cols + best]) best = j;
    wrong += best != lab[i];
  }
  return (float)wrong / (float)rows;
}

template <typename T>
void CrossEntropyLoss(const TinyTensor<T>& input, const TinyTensor<int>& labels, TinyTensor<T>& loss) {
  static_assert(std::is_same<T, float>::value, "CrossEntropyLoss is float only, as in the reference");
  const std::string fn = "CrossEntropyLoss";
  need_gpu(fn, "input", input.device);
  need_gpu(fn, "labels", labels.device);
  need_gpu(fn, "loss", loss.device);
  const auto [rows, cols] = ce_dims(fn, input, labels);
  no_alias(fn, {{input.p_data, "input"}}, {{loss.p_data, "loss"}});
  loss.resize(std::vector<int>{1});
  tt_check(tt_cross_entropy_f32(input.p_data, labels.p_data, loss.p_data, rows, cols, nullptr), fn.c_str());
  tt_check(tt_sync(), fn.c_str());
}

template <typename T>
void CrossEntropyLossBackward(const TinyTensor<T>& softmax_output, const TinyTensor<int>& labels,
                              TinyTensor<T>& grad_input) {
  static_assert(std::is_same<T, float>::value, "CrossEntropyLossBackward is float only, as in the reference");
  const std::string fn = "CrossEntropyLossBackward";
  need_gpu(fn, "softmax_output", softmax_output.device);
  need_gpu(fn, "labels", labels.device);
  need_gpu(fn, "grad_input", grad_input.device);
  const auto [rows, cols] = ce_dims(fn, softmax_output, labels);
  if (&grad_input != &softmax_output) grad_input.resize(softmax_output.shape);
  tt_check(tt_cross_entropy_backward_f32(softmax_output.p_data, labels.p_data, grad_input.p_data, rows, cols,
                                         nullptr),
           fn.c_str());
  tt_check(tt_sync(), fn.c_str());
}

template <typename T>
void MaxPoolingForward(const TinyTensor<T>& input, TinyTensor<T>& output, TinyTensor<T>& mask,
                       const std::vector<int>& kernel_shape, int pad_h, int pad_w, int stride_h, int stride_w) {
  static_assert(std::is_same<T, float>::value, "MaxPoolingForward is float only, as in the reference");
  const std::string fn = "MaxPoolingForward";
  need_gpu(fn, "input", input.device);
  need_gpu(fn, "output", output.device);
  need_gpu(fn, "mask", mask.device);
  if (kernel_shape.size() < 2) throw std::invalid_argument(fn + ": kernel_shape must end with [kh, kw]");
  const ConvShape s = conv_shape(fn, "input", input.shape);
  const int kh = kernel_shape[kernel_shape.size() - 2], kw = kernel_shape.back();
  const int oh = conv_out(fn, s.H, kh, pad_h, stride_h), ow = conv_out(fn, s.W, kw, pad_w, stride_w);
  no_alias(fn, {{input.p_data, "input"}}, {{output.p_data, "output"}, {mask.p_data, "mask"}});
  std::vector<int> oshape(input.shape.begin(), input.shape.end() - 2);
  oshape.insert(oshape.end(), {oh, ow});
  output.resize(oshape);
  mask.resize(oshape);
  tt_check(tt_maxpool_f32(input.p_data, output.p_data, mask.p_data, s.batch * s.C, s.H, s.W, kh, kw, pad_h, pad_w,
                          stride_h, stride_w, nullptr),
           fn.c_str());
  tt_check(tt_sync(), fn.c_str());
}

template <typename T>
void MaxPoolingBackward(const TinyTensor<T>& grad_output, const TinyTensor<T>& mask, TinyTensor<T>& grad_input,
                        const std::vector<int>& input_shape, const std::vector<int>& kernel_shape, int pad_h,
                        int pad_w, int stride_h, int stride_w) {
  static_assert(std::is_same<T, float>::value, "MaxPoolingBackward is float only, as in the reference");
  const std::string fn = "MaxPoolingBackward";
  need_gpu(fn, "grad_output", grad_output.device);
  need_gpu(fn, "mask", mask.device);
  need_gpu(fn, "grad_input", grad_input.device);
  if (kernel_shape.size() < 2) throw std::invalid_argument(fn + ": kernel_shape must end with [kh, kw]");
  if (input_shape.size() < 2) throw std::invalid_argument(fn + ": input_shape must end with [H, W]");
  const ConvShape go = conv_shape(fn, "grad_output", grad_output.shape);
  const int H = input_shape[input_shape.size() - 2], W = input_shape.back();
  const int kh = kernel_shape[kernel_shape.size() - 2], kw = kernel_shape.back();
  if (conv_out(fn, H, kh, pad_h, stride_h) != go.H || conv_out(fn, W, kw, pad_w, stride_w) != go.W)
    throw std::invalid_argument(fn + ": grad_output's last two axes do not match input_shape and the window");
  if (mask.size != grad_output.size) throw std::invalid_argument(fn + ": mask must have grad_output's shape");
  no_alias(fn, {{grad_output.p_data, "grad_output"}, {mask.p_data, "mask"}}, {{grad_input.p_data, "grad_input"}});
  // the reference's shape: grad_output's leading axes, then H, W (Layers.cu:301-315)
  std::vector<int> ishape(grad_output.shape.begin(), grad_output.shape.end() - 2);
  ishape.insert(ishape.end(), {H, W});
  grad_input.resize(ishape);
  tt_check(tt_maxpool_backward_f32(grad_output.p_data, mask.p_data, grad_input.p_data, go.batch * go.C, H, W, kh, kw,
                                   pad_h, pad_w, stride_h, stride_w, nullptr),
           fn.c_str());
  tt_check(tt_sync(), fn.c_str());
}

template void AttentionForward<float>(const TinyTensor<float>&, const TinyTensor<float>&, const TinyTensor<float>&,
                                      TinyTensor<float>&, TinyTensor<float>&, float, bool);
template void AttentionForward<bf16>(const TinyTensor<bf16>&, const TinyTensor<bf16>&, const TinyTensor<bf16>&,
                                     TinyTensor<bf16>&, TinyTensor<float>&, float, bool);
template void AttentionBackward<float>(const TinyTensor<float>&, const TinyTensor<float>&, const TinyTensor<float>&,
                                       const TinyTensor<float>&, const TinyTensor<float>&, const TinyTensor<float>&,
                                       TinyTensor<float>&, TinyTensor<float>&, TinyTensor<float>&, float, bool);
template void AttentionBackward<bf16>(const TinyTensor<bf16>&, const TinyTensor<bf16>&, const TinyTensor<bf16>&,
                                      const TinyTensor<bf16>&, const TinyTensor<float>&, const TinyTensor<bf16>&,
                                      TinyTensor<bf16>&, TinyTensor<bf16>&, TinyTensor<bf16>&, float, bool);
template void AttentionDecode<float>(const TinyTensor<float>&, const TinyTensor<float>&, const TinyTensor<float>&,
                                     TinyTensor<float>&, float);
template void AttentionDecode<bf16>(const TinyTensor<bf16>&, const TinyTensor<bf16>&, const TinyTensor<bf16>&,
                                    TinyTensor<bf16>&, float);
template void SoftmaxForward<float>(const TinyTensor<float>&, TinyTensor<float>&);
template void FcForward<float>(const TinyTensor<float>&, TinyTensor<float>&, const TinyTensor<float>&,
                               const TinyTensor<float>&);
template void FcForward<bf16>(const TinyTensor<bf16>&, TinyTensor<bf16>&, const TinyTensor<bf16>&,
                              const TinyTensor<bf16>&);
template void FcBackward<float>(const TinyTensor<float>&, const TinyTensor<float>&, const TinyTensor<float>&,
                                const TinyTensor<float>&, TinyTensor<float>&, const TinyTensor<float>&,
                                TinyTensor<float>&, TinyTensor<float>&);
template void FcBackward<bf16>(const TinyTensor<bf16>&, const TinyTensor<bf16>&, const TinyTensor<bf16>&,
                               const TinyTensor<bf16>&, TinyTensor<bf16>&, const TinyTensor<bf16>&,
                               TinyTensor<bf16>&, TinyTensor<bf16>&);
template void Im2col<float>(const TinyTensor<float>&, TinyTensor<float>&, const std::vector<int>&, int, int, int,
                            int);
template void Im2col<bf16>(const TinyTensor<bf16>&, TinyTensor<bf16>&, const std::vector<int>&, int, int, int, int);
template void Col2im<float>(const TinyTensor<float>&, TinyTensor<float>&, const std::vector<int>&,
                            const std::vector<int>&, int, int, int, int);
template void Col2im<bf16>(const TinyTensor<bf16>&, TinyTensor<bf16>&, const std::vector<int>&,
                           const std::vector<int>&, int, int, int, int);
template void ConvForward<float>(const TinyTensor<float>&, TinyTensor<float>&, const TinyTensor<float>&, int, int,
                                 int, int);
template void ConvForward<bf16>(const TinyTensor<bf16>&, TinyTensor<bf16>&, const TinyTensor<bf16>&, int, int, int,
                                int);
template void ConvBackward<float>(const TinyTensor<float>&, const TinyTensor<float>&, const TinyTensor<float>&,
                                  TinyTensor<float>&, const TinyTensor<float>&, TinyTensor<float>&, int, int, int,
                                  int);
template void ConvBackward<bf16>(const TinyTensor<bf16>&, const TinyTensor<bf16>&, const TinyTensor<bf16>&,
                                 TinyTensor<bf16>&, const TinyTensor<bf16>&, TinyTensor<bf16>&, int, int, int, int);
template float SoftmaxLoss<float>(const TinyTensor<float>&, const TinyTensor<int>&);
template void CrossEntropyLoss<float>(const TinyTensor<float>&, const TinyTensor<int>&, TinyTensor<float>&);
template void CrossEntropyLossBackward<float>(const TinyTensor<float>&, const TinyTensor<int>&, TinyTensor<float>&);
template void MaxPoolingForward<float>(const TinyTensor<float>&, TinyTensor<float>&, TinyTensor<float>&,
                                       const std::vector<int>&, int, int, int, int);
template void MaxPoolingBackward<float>(const TinyTensor<float>&, const TinyTensor<float>&, TinyTensor<float>&,
                                        const std::vector<int>&, const std::vector<int>&, int, int, int, int);
