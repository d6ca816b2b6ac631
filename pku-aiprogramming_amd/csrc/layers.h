// Attention, softmax and fully connected layer functions of the `myLayer` module.
//
// They follow the reference's layer convention (FcForward/FcBackward,
// Task3/Tinytensor/src/Layers.h:8-26, Layers.cu:9-79): inputs are const
// TinyTensor references on the "gpu" device, outputs are non-const
// references that the callee resizes in place (Layers.cu:25, 52-57), float
// instantiations plus bf16 ones for the attention path.
#pragma once

#include "tinytensor.h"

// O = softmax(scale * Q K^T + M) V and LSE (natural log, fp32 [B,H,Lq]).
// q [B,H,Lq,d], k/v [B,H,Lk,d]; causal -> M = -inf where key > query.
template <typename T>
void AttentionForward(const TinyTensor<T>& q, const TinyTensor<T>& k, const TinyTensor<T>& v,
                      TinyTensor<T>& out, TinyTensor<float>& lse, float scale, bool causal);

// dQ, dK, dV for upstream gradient grad_out from the saved out and lse.
template <typename T>
void AttentionBackward(const TinyTensor<T>& q, const TinyTensor<T>& k, const TinyTensor<T>& v,
                       const TinyTensor<T>& out, const TinyTensor<float>& lse,
                       const TinyTensor<T>& grad_out, TinyTensor<T>& grad_q, TinyTensor<T>& grad_k,
                       TinyTensor<T>& grad_v, float scale, bool causal);

// Single-query decode: q [B,H,1,d], caches [B,H,Lkv,d] -> out [B,H,1,d].
template <typename T>
void AttentionDecode(const TinyTensor<T>& q, const TinyTensor<T>& k_cache, const TinyTensor<T>& v_cache,
                     TinyTensor<T>& out, float scale);

// Row softmax over the last axis (Layers.cu:324-349): output takes input's
// shape on the "gpu" device (the reference's `output = input`, Layers.cu:333)
// and holds exp(x - max) / sum exp(x - max) per row.  float, as the
// reference binds it (bind_Layer.cpp:20); output may be input itself.
template <typename T>
void SoftmaxForward(const TinyTensor<T>& input, TinyTensor<T>& output);

// Fully connected layer (Layers.cu:9-39): output [.., fout] = input [.., fin]
// weight [fin, fout] + bias, every leading axis of input a batch axis.  bias
// is [fout], or [1] for one value added to every output (Layers.cu:28-33).
// The product runs on the library GEMM (tt_gemm_*, replacing cudaGemm); the
// bias is added by a rank-1 GEMM of a ones column against the bias row, as the
// reference does.  float as the reference binds it (bind_Layer.cpp:12-13),
// and bf16.
template <typename T>
void FcForward(const TinyTensor<T>& input, TinyTensor<T>& output, const TinyTensor<T>& weight,
               const TinyTensor<T>& bias);

// Its gradients (Layers.cu:41-79): grad_input = grad_output weight^T,
// grad_weight = input^T grad_output, grad_bias = the column sums of
// grad_output (their total for a [1] bias); each is resized to its operand's
// shape.  `output` is accepted and not read, as in the reference.
template <typename T>
void FcBackward(const TinyTensor<T>& input, const TinyTensor<T>& output, const TinyTensor<T>& weight,
                const TinyTensor<T>& bias, TinyTensor<T>& grad_input, const TinyTensor<T>& grad_output,
                TinyTensor<T>& grad_weight, TinyTensor<T>& grad_bias);

// Convolution data movement (Layers.cu:81-158): im [.., C, H, W] to its
// column matrix [P, C kh kw] (rank-3 image) or [batch, P, C kh kw], P = OH OW
// output pixels, and col2im, its adjoint, back to im_shape (each image
// element the sum of the column entries read from it).  kernel_shape's last
// two entries are kh, kw.
template <typename T>
void Im2col(const TinyTensor<T>& im_tensor, TinyTensor<T>& col_tensor, const std::vector<int>& kernel_shape,
            int pad_h, int pad_w, int stride_h, int stride_w);
template <typename T>
void Col2im(const TinyTensor<T>& col_tensor, TinyTensor<T>& im_tensor, const std::vector<int>& kernel_shape,
            const std::vector<int>& im_shape, int pad_h, int pad_w, int stride_h, int stride_w);

// Convolution layer (Layers.cu:160-200): input [.., Cin, H, W], weight
// [Cout, Cin, kh, kw] -> output [.., Cout, OH, OW]: one im2col launch for the
// batch, then per image output = weight (as [Cout, Cin kh kw]) col^T on the
// library GEMM.  No bias, as in the reference.
template <typename T>
void ConvForward(const TinyTensor<T>& input, TinyTensor<T>& output, const TinyTensor<T>& weight, int pad_h,
                 int pad_w, int stride_h, int stride_w);

// Its gradients (Layers.cu:202-252): grad_weight = sum over images of
// grad_output col (GEMM, accumulating), grad_col = grad_output^T weight per
// image, grad_input = col2im(grad_col).  `output` is accepted and not read.
template <typename T>
void ConvBackward(const TinyTensor<T>& input, const TinyTensor<T>& output, const TinyTensor<T>& weight,
                  TinyTensor<T>& grad_input, const TinyTensor<T>& grad_output, TinyTensor<T>& grad_weight,
                  int pad_h, int pad_w, int stride_h, int stride_w);

// Softmax cross-entropy after SoftmaxForward (Layers.cu:351-423), float as the
// reference binds them (bind_Layer.cpp:21-23).  input / softmax_output are
// softmax rows [.., classes], labels int [rows] on the "gpu" device.
// SoftmaxLoss: the fraction of rows whose first largest entry is not the
// label (computed on the host, as in the reference).  CrossEntropyLoss: loss
// [1] = sum of -log p[label] over the rows.  CrossEntropyLossBackward:
// grad_input = softmax_output - onehot(labels).
template <typename T>
float SoftmaxLoss(const TinyTensor<T>& softmax_output, const TinyTensor<int>& labels);
template <typename T>
void CrossEntropyLoss(const TinyTensor<T>& input, const TinyTensor<int>& labels, TinyTensor<T>& loss);
template <typename T>
void CrossEntropyLossBackward(const TinyTensor<T>& softmax_output, const TinyTensor<int>& labels,
                              TinyTensor<T>& grad_input);

// Max pooling (Layers.cu:254-322), float as the reference binds it: input
// [.., C, H, W] -> output and mask [.., C, OH, OW] (mask: the flat index of
// each window's first maximum in its plane); the backward routes grad_output
// to those elements of a grad_input of input_shape, summing where windows
// overlap.
template <typename T>
void MaxPoolingForward(const TinyTensor<T>& input, TinyTensor<T>& output, TinyTensor<T>& mask,
                       const std::vector<int>& kernel_shape, int pad_h, int pad_w, int stride_h, int stride_w);
template <typename T>
void MaxPoolingBackward(const TinyTensor<T>& grad_output, const TinyTensor<T>& mask, TinyTensor<T>& grad_input,
                        const std::vector<int>& input_shape, const std::vector<int>& kernel_shape, int pad_h,
                        int pad_w, int stride_h, int stride_w);

