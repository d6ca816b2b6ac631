// Module `myLayer`: the attention entry points, SoftmaxForward with its cross-entropy, FC, convolution and max pooling, bound in the style of
// Task3/Tinytensor/src/bind_Layer.cpp:10-24 (free functions over TinyTensor
// references), with float and bf16 overloads.
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include "layers.h"

namespace py = pybind11;

PYBIND11_MODULE(myLayer, m) {
  m.doc() = "myLayer: fused attention for MI355X (gfx950)";
  // The tensor classes are registered by myTensor; import it so that callers
  // can use myLayer first.
  py::module_::import("myTensor");
  m.def("AttentionForward", &AttentionForward<float>, py::arg("q"), py::arg("k"), py::arg("v"), py::arg("out"),
        py::arg("lse"), py::arg("scale"), py::arg("causal"));
  m.def("AttentionForward", &AttentionForward<bf16>, py::arg("q"), py::arg("k"), py::arg("v"), py::arg("out"),
        py::arg("lse"), py::arg("scale"), py::arg("causal"));
  m.def("AttentionBackward", &AttentionBackward<float>, py::arg("q"), py::arg("k"), py::arg("v"), py::arg("out"),
        py::arg("lse"), py::arg("grad_out"), py::arg("grad_q"), py::arg("grad_k"), py::arg("grad_v"),
        py::arg("scale"), py::arg("causal"));
  m.def("AttentionBackward", &AttentionBackward<bf16>, py::arg("q"), py::arg("k"), py::arg("v"), py::arg("out"),
        py::arg("lse"), py::arg("grad_out"), py::arg("grad_q"), py::arg("grad_k"), py::arg("grad_v"),
        py::arg("scale"), py::arg("causal"));
  m.def("AttentionDecode", &AttentionDecode<float>, py::arg("q"), py::arg("k_cache"), py::arg("v_cache"),
        py::arg("out"), py::arg("scale"));
  m.def("AttentionDecode", &AttentionDecode<bf16>, py::arg("q"), py::arg("k_cache"), py::arg("v_cache"),
        py::arg("out"), py::arg("scale"));
  // the reference binds SoftmaxForward<float> positionally (bind_Layer.cpp:20)
  m.def("SoftmaxForward", &SoftmaxForward<float>, py::arg("input"), py::arg("output"));
  // positional as in the reference (bind_Layer.cpp:12-13), plus bf16 overloads
  m.def("FcForward", &FcForward<float>, py::arg("input"), py::arg("output"), py::arg("weight"), py::arg("bias"));
  m.def("FcForward", &FcForward<bf16>, py::arg("input"), py::arg("output"), py::arg("weight"), py::arg("bias"));
  m.def("FcBackward", &FcBackward<float>, py::arg("input"), py::arg("output"), py::arg("weight"), py::arg("bias"),
        py::arg("grad_input"), py::arg("grad_output"), py::arg("grad_weight"), py::arg("grad_bias"));
  m.def("FcBackward", &FcBackward<bf16>, py::arg("input"), py::arg("output"), py::arg("weight"), py::arg("bias"),
        py::arg("grad_input"), py::arg("grad_output"), py::arg("grad_weight"), py::arg("grad_bias"));
  m.def("MaxPoolingForward", &MaxPoolingForward<float>, py::arg("input"), py::arg("output"), py::arg("mask"),
        py::arg("kernel_shape"), py::arg("pad_h"), py::arg("pad_w"), py::arg("stride_h"), py::arg("stride_w"));
  m.def("MaxPoolingBackward", &MaxPoolingBackward<float>, py::arg("grad_output"), py::arg("mask"),
        py::arg("grad_input"), py::arg("input_shape"), py::arg("kernel_shape"), py::arg("pad_h"), py::arg("pad_w"),
        py::arg("stride_h"), py::arg("stride_w"));
  // float, positional, as the reference binds them (bind_Layer.cpp:21-23)
  m.def("SoftmaxLoss", &SoftmaxLoss<float>, py::arg("softmax_output"), py::arg("labels"));
  m.def("CrossEntropyLoss", &CrossEntropyLoss<float>, py::arg("input"), py::arg("labels"), py::arg("loss"));
  m.def("CrossEntropyLossBackward", &CrossEntropyLossBackward<float>, py::arg("softmax_output"), py::arg("labels"),
        py::arg("grad_input"));
  // the reference's names and argument order (bind_Layer.cpp:14-17), plus bf16 overloads
  m.def("im2col", &Im2col<float>, py::arg("im_tensor"), py::arg("col_tensor"), py::arg("kernel_shape"),
        py::arg("pad_h"), py::arg("pad_w"), py::arg("stride_h"), py::arg("stride_w"));
  m.def("im2col", &Im2col<bf16>, py::arg("im_tensor"), py::arg("col_tensor"), py::arg("kernel_shape"),
        py::arg("pad_h"), py::arg("pad_w"), py::arg("stride_h"), py::arg("stride_w"));
  m.def("col2im", &Col2im<float>, py::arg("col_tensor"), py::arg("im_tensor"), py::arg("kernel_shape"),
        py::arg("im_shape"), py::arg("pad_h"), py::arg("pad_w"), py::arg("stride_h"), py::arg("stride_w"));
  m.def("col2im", &Col2im<bf16>, py::arg("col_tensor"), py::arg("im_tensor"), py::arg("kernel_shape"),
        py::arg("im_shape"), py::arg("pad_h"), py::arg("pad_w"), py::arg("stride_h"), py::arg("stride_w"));
  m.def("ConvForward", &ConvForward<float>, py::arg("input"), py::arg("output"), py::arg("weight"),
        py::arg("pad_h"), py::arg("pad_w"), py::arg("stride_h"), py::arg("stride_w"));
  m.def("ConvForward", &ConvForward<bf16>, py::arg("input"), py::arg("output"), py::arg("weight"),
        py::arg("pad_h"), py::arg("pad_w"), py::arg("stride_h"), py::arg("stride_w"));
  m.def("ConvBackward", &ConvBackward<float>, py::arg("input"), py::arg("output"), py::arg("weight"),
        py::arg("grad_input"), py::arg("grad_output"), py::arg("grad_weight"), py::arg("pad_h"), py::arg("pad_w"),
        py::arg("stride_h"), py::arg("stride_w"));
  m.def("ConvBackward", &ConvBackward<bf16>, py::arg("input"), py::arg("output"), py::arg("weight"),
        py::arg("grad_input"), py::arg("grad_output"), py::arg("grad_weight"), py::arg("pad_h"), py::arg("pad_w"),
        py::arg("stride_h"), py::arg("stride_w"));
}
