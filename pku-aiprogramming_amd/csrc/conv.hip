// im2col / col2im: the data movement of the convolution layer on the library
// GEMM (reference src/Layers.cu:81-158, kernels src/Layers_kernels.cu:32-105).
//
// Layout (the reference's): an image batch im[N][C][H][W] and its column
// matrix col[N][P][C][kh][kw], P = OH * OW output pixels in row-major order,
//   col[n][oy * OW + ox][c][ky][kx] = im[n][c][oy sh - ph + ky][ox sw - pw + kx]
// (0 outside the image), OH = (H + 2 ph - kh) / sh + 1, OW likewise.  col2im
// is its adjoint: every image element is the sum of the column entries that
// read it.  Both kernels gather (one thread per output element, a fixed
// order of the sums, no atomics), the whole batch in one launch.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "tt_internal.h"

namespace tt {

namespace {

struct ConvGeom {
  int C, H, W, kh, kw, ph, pw, sh, sw, oh, ow;
};

__device__ __forceinline__ float to_f(float x) { return x; }
__device__ __forceinline__ float to_f(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }
__device__ __forceinline__ void from_f(float v, float& out) { out = v; }
__device__ __forceinline__ void from_f(float v, uint16_t& out) {
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    out = uint16_t((u >> 16) | 0x40);  // quiet NaN
    return;
  }
  u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest even
  out = uint16_t(u >> 16);
}

// One thread per column entry (n, p, c, ky, kx), in the column's order, so
// that consecutive threads write consecutive elements.
template <typename T>
__global__ __launch_bounds__(256) void k_im2col(const T* __restrict__ im, T* __restrict__ col, int64_t total,
                                                ConvGeom g) {
  const int64_t P = (int64_t)g.oh * g.ow;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    int64_t r = i;
    const int kx = (int)(r % g.kw);
    r /= g.kw;
    const int ky = (int)(r % g.kh);
    r /= g.kh;
    const int c = (int)(r % g.C);
    r /= g.C;
    const int64_t p = r % P, n = r / P;
    const int oy = (int)(p / g.ow), ox = (int)(p % g.ow);
    const int y = oy * g.sh - g.ph + ky, x = ox * g.sw - g.pw + kx;
    T v = T(0);
    if (y >= 0 && y < g.H && x >= 0 && x < g.W) v = im[((n * g.C + c) * g.H + y) * g.W + x];
    col[i] = v;
  }
}

// One thread per image element (n, c, y, x): the sum, in float, of the column
// entries (oy, ox, ky, kx) with oy sh - ph + ky = y and ox sw - pw + kx = x,
// ky and kx ascending.
template <typename T>
__global__ __launch_bounds__(256) void k_col2im(const T* __restrict__ col, T* __restrict__ im, int64_t total,
                                                ConvGeom g) {
  const int64_t K = (int64_t)g.C * g.kh * g.kw;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    int64_t r = i;
    const int x = (int)(r % g.W);
    r /= g.W;
    const int y = (int)(r % g.H);
    r /= g.H;
    const int c = (int)(r % g.C);
    const int64_t n = r / g.C;
    const T* cn = col + n * (int64_t)g.oh * g.ow * K + (int64_t)c * g.kh * g.kw;
    float s = 0.f;
    for (int ky = 0; ky < g.kh; ++ky) {
      const int ty = y + g.ph - ky;
      if (ty < 0 || ty % g.sh != 0) continue;
      const int oy = ty / g.sh;
      if (oy >= g.oh) continue;
      for (int kx = 0; kx < g.kw; ++kx) {
        const int tx = x + g.pw - kx;
        if (tx < 0 || tx % g.sw != 0) continue;
        const int ox = tx / g.sw;
        if (ox >= g.ow) continue;
        s += to_f(cn[((int64_t)oy * g.ow + ox) * K + ky * g.kw + kx]);
      }
    }
    from_f(s, im[i]);
  }
}

// Max pooling (reference src/Layers.cu:254-322, kernels
// src/Layers_kernels.cu:109-175): one thread per output element; the window
// is clipped to the image (padding never wins), the first largest entry in
// row-major order is kept, and mask holds its index y * W + x in the (n, c)
// plane as a float (-1, and -FLT_MAX out, for a window with no image element).
__global__ __launch_bounds__(256) void k_maxpool(const float* __restrict__ in, float* __restrict__ out,
                                                 float* __restrict__ mask, int64_t total, ConvGeom g) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int ox = (int)(i % g.ow), oy = (int)((i / g.ow) % g.oh);
    const int64_t plane = i / ((int64_t)g.oh * g.ow);
    const int y0 = oy * g.sh - g.ph, x0 = ox * g.sw - g.pw;
    const int y1 = min(y0 + g.kh, g.H), x1 = min(x0 + g.kw, g.W);
    const float* pl = in + plane * g.H * g.W;
    float best = -3.402823466e38f;
    int arg = -1;
    for (int y = max(y0, 0); y < y1; ++y)
      for (int x = max(x0, 0); x < x1; ++x)
        if (pl[y * g.W + x] > best) {
          best = pl[y * g.W + x];
          arg = y * g.W + x;
        }
    out[i] = best;
    mask[i] = (float)arg;
  }
}

// Its gradient, one thread per input element: the sum of grad_out over the
// windows whose mask points at this element (the reference assigns instead,
// which with overlapping windows keeps one of them, whichever thread writes
// last; with non-overlapping windows the two agree).
__global__ __launch_bounds__(256) void k_maxpool_backward(const float* __restrict__ gout,
                                                          const float* __restrict__ mask,
                                                          float* __restrict__ gin, int64_t total, ConvGeom g) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int x = (int)(i % g.W), y = (int)((i / g.W) % g.H);
    const int64_t plane = i / ((int64_t)g.H * g.W);
    const float* gp = gout + plane * g.oh * g.ow;
    const float* mp = mask + plane * g.oh * g.ow;
    const float self = (float)(y * g.W + x);
    float s = 0.f;
    for (int ky = 0; ky < g.kh; ++ky) {
      const int ty = y + g.ph - ky;
      if (ty < 0 || ty % g.sh != 0 || ty / g.sh >= g.oh) continue;
      for (int kx = 0; kx < g.kw; ++kx) {
        const int tx = x + g.pw - kx;
        if (tx < 0 || tx % g.sw != 0 || tx / g.sw >= g.ow) continue;
        const int o = (ty / g.sh) * g.ow + tx / g.sw;
        if (mp[o] == self) s += gp[o];
      }
    }
    gin[i] = s;
  }
}

int conv_geom(const char* fn, int64_t N, int C, int H, int W, int kh, int kw, int ph, int pw, int sh, int sw,
              ConvGeom& g) {
  if (N < 0 || C < 1 || H < 1 || W < 1 || kh < 1 || kw < 1)
    return fail(TT_ERR_ARG, std::string(fn) + ": N >= 0 and C, H, W, kernel sizes >= 1 required");
  if (ph < 0 || pw < 0 || sh < 1 || sw < 1)
    return fail(TT_ERR_ARG, std::string(fn) + ": pads >= 0 and strides >= 1 required");
  if ((int64_t)H + 2 * (int64_t)ph < kh || (int64_t)W + 2 * (int64_t)pw < kw)
    return fail(TT_ERR_ARG, std::string(fn) + ": the kernel is larger than the padded image");
  g = ConvGeom{C, H, W, kh, kw, ph, pw, sh, sw, (int)((H + 2 * (int64_t)ph - kh) / sh + 1),
               (int)((W + 2 * (int64_t)pw - kw) / sw + 1)};
  return TT_OK;
}

template <typename T, bool TO_COL>
int conv_move(const char* fn, const void* src, void* dst, int64_t N, const ConvGeom& g, void* stream) {
  const int64_t total = TO_COL ? N * g.oh * g.ow * (int64_t)g.C * g.kh * g.kw : N * (int64_t)g.C * g.H * g.W;
  if (total == 0) return ok();
  if (!src || !dst) return fail(TT_ERR_ARG, std::string(fn) + ": null pointer");
  int rc = ensure_init();
  if (rc) return rc;
  hipStream_t s = stream_or_default(stream);
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;  // grid-stride beyond
  if (TO_COL)
    hipLaunchKernelGGL(k_im2col<T>, dim3((unsigned)blocks), dim3(256), 0, s, (const T*)src, (T*)dst, total, g);
  else
    hipLaunchKernelGGL(k_col2im<T>, dim3((unsigned)blocks), dim3(256), 0, s, (const T*)src, (T*)dst, total, g);
  TT_LAUNCHED(fn, s);
  return ok();
}

template <bool TO_COL>
int conv_entry(const char* fn, int dtype, const void* src, void* dst, int64_t N, int C, int H, int W, int kh,
               int kw, int ph, int pw, int sh, int sw, void* stream) {
  ConvGeom g;
  int rc = conv_geom(fn, N, C, H, W, kh, kw, ph, pw, sh, sw, g);
  if (rc) return rc;
  if (dtype == TT_F32) return conv_move<float, TO_COL>(fn, src, dst, N, g, stream);
  if (dtype == TT_BF16) return conv_move<uint16_t, TO_COL>(fn, src, dst, N, g, stream);
  return fail(TT_ERR_ARG, std::string(fn) + ": dtype must be TT_F32 or TT_BF16");
}

}  // namespace

}  // namespace tt

using namespace tt;

extern "C" int tt_im2col(int dtype, const void* im, void* col, int64_t N, int C, int H, int W, int kh, int kw,
                         int pad_h, int pad_w, int stride_h, int stride_w, void* stream) {
  return conv_entry<true>("tt_im2col", dtype, im, col, N, C, H, W, kh, kw, pad_h, pad_w, stride_h, stride_w, stream);
}

extern "C" int tt_col2im(int dtype, const void* col, void* im, int64_t N, int C, int H, int W, int kh, int kw,
                         int pad_h, int pad_w, int stride_h, int stride_w, void* stream) {
  return conv_entry<false>("tt_col2im", dtype, col, im, N, C, H, W, kh, kw, pad_h, pad_w, stride_h, stride_w,
                           stream);
}

namespace tt {
namespace {

// backward: (a, b, c) = (grad_out, mask, grad_in); forward: (in, out, mask).
int pool_launch(const char* fn, bool backward, const float* a, float* b, float* c, int64_t planes, int H, int W,
                int kh, int kw, int ph, int pw, int sh, int sw, void* stream) {
  ConvGeom g;
  int rc = conv_geom(fn, planes, 1, H, W, kh, kw, ph, pw, sh, sw, g);
  if (rc) return rc;
  const int64_t total = backward ? planes * (int64_t)H * W : planes * (int64_t)g.oh * g.ow;
  if (total == 0) return ok();
  if (!a || !b || !c) return fail(TT_ERR_ARG, std::string(fn) + ": null pointer");
  rc = ensure_init();
  if (rc) return rc;
  hipStream_t s = stream_or_default(stream);
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (backward)
    hipLaunchKernelGGL(k_maxpool_backward, dim3((unsigned)blocks), dim3(256), 0, s, a, b, c, total, g);
  else
    hipLaunchKernelGGL(k_maxpool, dim3((unsigned)blocks), dim3(256), 0, s, a, b, c, total, g);
  TT_LAUNCHED(fn, s);
  return ok();
}

}  // namespace
}  // namespace tt

extern "C" int tt_maxpool_f32(const float* in, float* out, float* mask, int64_t planes, int H, int W, int kh,
                              int kw, int pad_h, int pad_w, int stride_h, int stride_w, void* stream) {
  return tt::pool_launch("tt_maxpool_f32", false, in, out, mask, planes, H, W, kh, kw, pad_h, pad_w, stride_h,
                         stride_w, stream);
}

extern "C" int tt_maxpool_backward_f32(const float* grad_out, const float* mask, float* grad_in, int64_t planes,
                                       int H, int W, int kh, int kw, int pad_h, int pad_w, int stride_h,
                                       int stride_w, void* stream) {
  // the mask is only read; the helper's middle pointer is writable for the forward's output
  return tt::pool_launch("tt_maxpool_backward_f32", true, grad_out, const_cast<float*>(mask), grad_in, planes, H, W,
                         kh, kw, pad_h, pad_w, stride_h, stride_w, stream);
}

