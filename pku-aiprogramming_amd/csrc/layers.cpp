// Attention and softmax layer functions: shape checks, output sizing, then one C-ABI call.
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
