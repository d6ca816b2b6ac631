/*
 * tt_attn.h -- C-ABI of the MI355X (gfx950) TinyTensor runtime and its
 * scaled dot-product attention kernels.
 *
 * Every function returns an int status (TT_OK = 0).  On failure the message
 * is available from tt_last_error() (thread-local).  No C++ exception crosses
 * this boundary and no type here is a PyTorch or HIP type: pointers are plain
 * device addresses obtained from tt_malloc, sizes are int64_t / size_t, and a
 * stream argument of NULL means the library's own stream (tt_stream()).
 *
 * Reference interfaces replaced (csxq0605/pku-aiprogramming, Task3/Tinytensor):
 *   storage      cudaMalloc / cudaFree / cudaMemcpy / cudaMemset calls inside
 *                TinyTensor<T> (src/Tinytensor.cu:21,39-40,60-61,77-78,90,
 *                125,189,213,238,251-252,300,376-378)
 *   elementwise  the grid-stride kernels of src/TinyTensor_kernels.cu:6-85
 *                (launched at src/Tinytensor.cu:145,167,281,308,322,336,350,
 *                393,422,427,443,474,479)
 *   attention    the composition O = softmax((Q @ K^T) * s + M) @ V of
 *                optimizer/operators.py:163-164,181-182,234-242,194-199,
 *                611-612,416-433 (forward) and the gradient rules the autodiff
 *                driver runs over it (optimizer/autodiff.py:33-61), whose GPU
 *                row-softmax stage is SoftmaxForward (src/Layers.cu:324-349).
 *
 * Tensor layout: contiguous row-major [B, H, L, d] (TinyTensor has no
 * strides, src/Tinytensor.cu:47-66).  bf16 tensors are uint16_t bit patterns.
 * LSE is float32 [B, H, Lq], natural log.
 */
#ifndef TT_ATTN_H
#define TT_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  TT_OK = 0,
  TT_ERR_ARG = 1,         /* invalid argument (shape, null pointer, dtype) */
  TT_ERR_HIP = 2,         /* a HIP runtime call failed */
  TT_ERR_UNSUPPORTED = 3, /* valid but not implemented (e.g. head dim 96) */
  TT_ERR_NOMEM = 4        /* device allocation failed */
};

/* dtype codes for the generic entry points */
enum { TT_F32 = 0, TT_F64 = 1, TT_I32 = 2, TT_BF16 = 3 };

/* ---------------------------------------------------------------- runtime */

/* Message of the last failed call on this thread ("" if none). */
const char* tt_last_error(void);
/* Library version string. */
const char* tt_version(void);
/* Number of visible HIP devices (0 without a GPU; never fails). */
int tt_device_count(int* n);
/* Select the device and create the library stream (idempotent). */
int tt_init(int device);
/* The library stream as an opaque handle (hipStream_t). */
void* tt_stream(void);

/* Caller streams (no counterpart in the reference, which launches on the
 * default stream and synchronises after every launch): a new non-blocking
 * stream of default priority, a wait for all work queued on a stream (NULL:
 * the library stream), and its destruction (after waiting for it and
 * releasing the library's per-stream scratch buffers).  Every launcher takes
 * such a stream; two calls on different streams share no scratch memory. */
int tt_stream_create(void** stream);
int tt_stream_sync(void* stream);
int tt_stream_destroy(void* stream);

/* Caching device allocator (hipMalloc-backed).
 * Replaces cudaMalloc at src/Tinytensor.cu:21,39,60,77,116,252,375.
 * Blocks are reused by size class; tt_empty_cache() returns them (and the
 * launchers' scratch buffers) to HIP.  A refused allocation is TT_ERR_NOMEM;
 * with TT_FAIL_ALLOC_AFTER=n in the environment, the process's device
 * allocations n, n+1, ... are refused (failure injection for tests). */
int tt_malloc(void** ptr, size_t bytes);
/* Replaces cudaFree at src/Tinytensor.cu:90,108,239,378.  NULL is a no-op.
 * Unlike cudaFree it does not wait for the device: the block goes back to
 * the cache at once, and its next owner's work is ordered after the freed
 * block's last use only when both run on the library stream.  Work queued
 * on a caller stream that still reads or writes the block must have
 * finished (tt_stream_sync) before the block is freed. */
int tt_free(void* ptr);
int tt_empty_cache(void);
/* Bytes currently handed out / held in the cache. */
int tt_mem_stats(size_t* in_use, size_t* cached);

/* Copies ordered on the library stream.  d2h and h2d return after the copy
 * completed (the reference's copies are synchronous: src/Tinytensor.cu:40,61,
 * 213,238,251).  d2d is stream-ordered (src/Tinytensor.cu:78,125,189,377).
 * h2d / d2h of 4 MiB or more from pageable host memory run through pinned
 * staging buffers (16 MiB x 3, allocated on first use and kept), copied by
 * up to TT_HOST_THREADS host threads (default min(16, CPUs in the process's
 * affinity mask)) while the DMA engine moves the previous chunk; pinned host
 * memory is copied directly. */
int tt_memcpy_h2d(void* dst, const void* src, size_t bytes);
int tt_memcpy_d2h(void* dst, const void* src, size_t bytes);
int tt_memcpy_d2d(void* dst, const void* src, size_t bytes);
/* Converting copies for bf16 storage (no counterpart in the reference, which
 * has no bf16 tensors; they replace its upload/download of host values,
 * src/Tinytensor.cu:40,213): n float32 host values rounded to nearest even
 * into n bf16 on the device (NaN stays NaN), and n device bf16 widened into
 * float32 host values.  The conversion runs in the staging pass above;
 * synchronous like tt_memcpy_h2d / tt_memcpy_d2h. */
int tt_upload_bf16_from_f32(void* dst, const float* src, size_t n);
int tt_download_bf16_to_f32(float* dst, const void* src, size_t n);
/* Pinned (page-locked) host memory, as cudaMallocHost / cudaFreeHost (the
 * reference allocates none; it is here so that callers can hand
 * tt_memcpy_h2d / tt_memcpy_d2h memory the DMA engine reads directly).
 * tt_host_free(NULL) is a no-op. */
int tt_host_malloc(void** ptr, size_t bytes);
int tt_host_free(void* ptr);
/* Byte fill (src/Tinytensor.cu:300 cudaMemset). */
int tt_memset(void* ptr, int value, size_t bytes);
/* Wait for all work on the library stream. */
int tt_sync(void);

/* Stream-ordered timing events (hipEvent) for benchmarks. */
int tt_event_create(void** ev);
int tt_event_record(void* ev, void* stream);
int tt_event_elapsed_ms(float* ms, void* start, void* stop);
int tt_event_destroy(void* ev);

/* Benchmark instrumentation (no counterpart in the reference): after this
 * call the library records evs[i] on the launch stream right after its i-th
 * kernel launch, for i < n; later launches record nothing.  n = 0 (or
 * evs = NULL) disables it.  The events must stay alive until recorded. */
int tt_set_launch_events(void** evs, int n);
/* How many of those events the launches since tt_set_launch_events have
 * recorded (a step whose kernel count depends on the shape, such as the
 * decode with one or two launches, is timed by the events it recorded). */
int tt_launch_events_recorded(int* n);

/* Benchmark instrumentation (no counterpart in the reference): streams
 * `bytes` bytes of device memory at `buf` (16-byte aligned, bytes a multiple
 * of 16) with 16-byte non-temporal loads, one contiguous 256 KiB run per workgroup, and
 * stores nothing (out, one float, is written only if the data sums to a
 * sentinel).  It gives the HBM read rate that the decode kernel, which also
 * streams K and V once, is compared against. */
int tt_read_probe(const void* buf, int64_t bytes, float* out, void* stream);

/* ------------------------------------------------------------ elementwise */

/* Elementwise ops of TinyTensor (src/TinyTensor_kernels.cu:6-85).
 * op codes:
 *   TT_EW_ADD  c = a + b            cudaAdd        (:6-11)
 *   TT_EW_SUB  c = a - b            cudaSub        (:13-18)
 *   TT_EW_FILL c = alpha            cudaOnes/cudaFloatks (:30-35, :51-56)
 *   TT_EW_NEG  c = -a               cudaNegative   (:37-42)
 *   TT_EW_SCALE c = a * alpha       cudaMults      (:44-49)
 *   TT_EW_RELU c = max(a, 0)        Relu_Forward   (:58-63)
 *   TT_EW_RELU_BWD c = a>0 ? b : 0  Relu_Backward  (:65-70)
 *   TT_EW_SIGMOID c = 1/(1+e^-a)    Sigmoid_Forward (:72-77)
 *   TT_EW_SIGMOID_BWD c = s(a)(1-s(a)) b  Sigmoid_Backward (:79-85)
 *   TT_EW_UNIFORM c ~ U[alpha, beta) from a counter hash of (seed, index)
 *                                   cudaRandom     (:20-28)
 * a, b may be NULL where unused; c may alias a.  n is the element count. */
enum {
  TT_EW_ADD = 0, TT_EW_SUB = 1, TT_EW_FILL = 2, TT_EW_NEG = 3, TT_EW_SCALE = 4,
  TT_EW_RELU = 5, TT_EW_RELU_BWD = 6, TT_EW_SIGMOID = 7, TT_EW_SIGMOID_BWD = 8,
  TT_EW_UNIFORM = 9
};
int tt_elementwise(int op, int dtype, void* c, const void* a, const void* b, int64_t n,
                   double alpha, double beta, uint64_t seed, void* stream);

/* Fill a bf16 / fp32 buffer with scale * N(0,1) samples from a counter-based
 * generator (SplitMix64 of (seed, index) -> Box-Muller).  Synthetic benchmark
 * data only; not part of the reference. */
int tt_fill_normal(int dtype, void* dst, int64_t n, uint64_t seed, float scale, void* stream);

/* ------------------------------------------------------------- attention */

/* For every attention launcher below: an output whose bytes overlap an
 * input's or another output's is refused with TT_ERR_ARG before anything is
 * launched (the kernels read their inputs while writing their outputs);
 * inputs may overlap each other (q == k == v is a valid call). */

/* Forward: O = softmax(scale * Q K^T + M) V, LSE = rowwise log-sum-exp of the
 * scaled, masked scores (natural log).  M is the strict upper triangle
 * (key j > query i, top-left aligned) when causal != 0, else nothing.
 * q [B,H,Lq,d], k/v [B,H,Lk,d], o [B,H,Lq,d], lse [B,H,Lq] (may be NULL).
 * d in {32, 64, 128}; causal requires Lq == Lk; Lk >= 1 when Lq >= 1.
 * Replaces the composition at optimizer/operators.py:163-164 (Q @ K^T),
 * :234-239 (* s), :194-196 (+ mask), :611-612 (softmax), :416-419 (@ V).
 * The bf16 forward allocates nothing.  The fp32 forward of a problem with
 * fewer query tiles than the GPU has workgroup slots splits the keys and
 * merges partial results through a per-stream library workspace (allocated
 * on first use, TT_ERR_NOMEM if that fails). */
int tt_attn_fwd_f32(const float* q, const float* k, const float* v, float* o, float* lse,
                    int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t d,
                    float scale, int causal, void* stream);
int tt_attn_fwd_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o,
                     float* lse, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t d,
                     float scale, int causal, void* stream);

/* Backward of the forward above for upstream gradient do_ (same shape as o),
 * from the saved o and lse:  D = rowsum(dO o O); P recomputed from LSE;
 * dV = P^T dO; dP = dO V^T; dS = P o (dP - D); dQ = s dS K; dK = s dS^T Q.
 * Replaces O.backward(dO) (optimizer/operators.py:115-119 -> autodiff.py:33-61)
 * through MatMul.gradient (:421-429), Transpose.gradient (:338-340),
 * MulScalar.gradient (:241-242), EWiseDiv.gradient (:296-298),
 * BroadcastTo/Summation.gradient (:373-380, :400-408), Exp.gradient (:469-470).
 * No L x L matrix is stored: one kernel owns dK/dV rows (keys) and one owns
 * dQ rows (queries), and each recomputes S and dP from Q, K, V, dO and the
 * LSE.  Uses a library-owned scratch buffer of 2*B*H*Lq floats (-D and
 * LSE*log2(e)), one per stream. */
int tt_attn_bwd_f32(const float* q, const float* k, const float* v, const float* o,
                    const float* lse, const float* do_, float* dq, float* dk, float* dv,
                    int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t d,
                    float scale, int causal, void* stream);
int tt_attn_bwd_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                     const uint16_t* o, const float* lse, const uint16_t* do_,
                     uint16_t* dq, uint16_t* dk, uint16_t* dv,
                     int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t d,
                     float scale, int causal, void* stream);

/* Allocation-free variant of tt_attn_bwd_bf16 (same arguments, kernels and
 * results).  It has no counterpart in the reference; it is for callers that
 * cannot allocate device memory: code under HIP graph capture, tight serving
 * or training loops, harnesses that forbid hipMalloc.  Its row scratch (-D
 * and LSE*log2(e), 8 bytes per query row) is a 16 MiB static device array per
 * GPU, so B*H*Lq must not exceed 2097152 rows (TT_ERR_ARG beyond).  It calls
 * no allocator and does no set-up: tt_init must have run (TT_ERR_ARG
 * otherwise).  Every call on one GPU shares that array: calls that overlap
 * on one GPU (two streams, or two host threads) race; order them.  The
 * array keeps the last call's contents; each call writes every row it reads
 * before reading it. */
int tt_attn_bwd_bf16_noalloc(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                             const uint16_t* o, const float* lse, const uint16_t* do_,
                             uint16_t* dq, uint16_t* dk, uint16_t* dv,
                             int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t d,
                             float scale, int causal, void* stream);

/* Single-query decode: o = softmax(scale * q K^T) V per (b, h), no mask.
 * q [B,H,1,d], k/v cache [B,H,Lkv,d] contiguous, o [B,H,1,d], lse [B,H] (may
 * be NULL).  The same composition as the forward with Lq = 1 (a3 -> a4 -> a6
 * -> a7 of the reference's op chain).  Splits Lkv across workgroups and merges
 * the partial (o, lse) pairs by LSE rescaling; partials live in a
 * library-owned scratch buffer. */
int tt_attn_decode_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o,
                        float* lse, int64_t B, int64_t H, int64_t Lkv, int64_t d,
                        float scale, void* stream);
int tt_attn_decode_f32(const float* q, const float* k, const float* v, float* o, float* lse,
                       int64_t B, int64_t H, int64_t Lkv, int64_t d, float scale,
                       void* stream);

/* ------------------------------------------------------------- softmax */

/* Row softmax over the last axis of a row-major [rows, cols] fp32 matrix:
 *   y[r][c] = exp(x[r][c] - m_r) / sum_c' exp(x[r][c'] - m_r),  m_r = max_c x[r][c].
 * Replaces SoftmaxForward (src/Layers.cu:324-349: cudaChannelMax, Sub, Exp,
 * Sum, Div of src/Layers_kernels.cu:189-257, the max and the sum each a host
 * loop of thrust calls per row) with one kernel that reads each element once
 * into registers and writes it once: a wave per row up to 2048 columns, a
 * workgroup per row up to 8192 (65536 for rows that are not 16-byte
 * aligned), and for aligned rows of 8196 .. 2 Mi columns 2-64 workgroups per
 * row that merge their (max, sum) partials through a per-stream library
 * workspace of rows x chunks x 16 bytes (allocated on first use,
 * TT_ERR_NOMEM if that fails; calls on one stream share it in order).
 * Longer rows are read twice.  y may alias x.  A row of -inf (or holding
 * +inf or NaN) gives NaN, as the reference's x - max does. */
int tt_softmax_rows_f32(const float* x, float* y, int64_t rows, int64_t cols, void* stream);

/* loss[0] = sum over rows i of -log p[i][labels[i]] for softmax rows p
 * [rows x cols] and int labels: the reference's CrossEntropyLoss
 * (src/Layers.cu:383-404; kernel src/Layers_kernels.cu:260-270, then a
 * thrust sum), in double, in a fixed order.  A label outside [0, cols) gives
 * NaN.  The caller synchronizes before reading loss. */
int tt_cross_entropy_f32(const float* p, const int* labels, float* loss, int64_t rows, int64_t cols, void* stream);
/* grad = p - onehot(labels) (rows x cols), the reference's
 * CrossEntropyLossBackward (src/Layers.cu:406-423); a label outside [0, cols)
 * subtracts nothing.  grad may alias p. */
int tt_cross_entropy_backward_f32(const float* p, const int* labels, float* grad, int64_t rows, int64_t cols,
                                  void* stream);

/* ---------------------------------------------------------------- GEMM */

/* C = alpha op(A) op(B) + beta C, all row-major: op(A) is m x k, op(B) is
 * k x n, C is m x n (ldc = n).  transa = 0: A stored m x k (lda = k); 1: A
 * stored k x m (lda = m).  transb = 0: B stored k x n (ldb = n); 1: B stored
 * n x k (ldb = k).  beta = 0 does not read C.  Replaces cudaGemm
 * (src/Layers_kernels.cu:10-30: a cuBLAS handle created and destroyed around
 * one cublasSgemm per call), called by FcForward / FcBackward (src/Layers.cu:
 * 26-77) and ConvForward / ConvBackward (:197, :247-248).  fp32: fp32
 * products and sums on the fp32 MFMA; bf16: bf16 A, B, C with fp32 sums. */
int tt_gemm_f32(int transa, int transb, int64_t m, int64_t n, int64_t k, float alpha,
                const float* A, const float* B, float beta, float* C, void* stream);
int tt_gemm_bf16(int transa, int transb, int64_t m, int64_t n, int64_t k, float alpha,
                 const uint16_t* A, const uint16_t* B, float beta, uint16_t* C, void* stream);

/* ---------------------------------------------------------------- convolution data movement */

/* im[N][C][H][W] -> col[N][OH*OW][C][kh][kw] with OH = (H + 2 pad_h - kh) /
 * stride_h + 1 (OW likewise), col[n][oy*OW + ox][c][ky][kx] =
 * im[n][c][oy stride_h - pad_h + ky][ox stride_w - pad_w + kx] and 0 outside
 * the image: the reference's im2col (src/Layers.cu:81-119, kernel
 * src/Layers_kernels.cu:32-66, one launch per batch image), here one launch
 * for the batch.  dtype TT_F32 or TT_BF16. */
int tt_im2col(int dtype, const void* im, void* col, int64_t N, int C, int H, int W, int kh, int kw, int pad_h,
              int pad_w, int stride_h, int stride_w, void* stream);
/* Its adjoint, the reference's col2im (src/Layers.cu:121-158, kernel
 * src/Layers_kernels.cu:68-105): im[n][c][y][x] = the sum (in fp32) of the
 * col entries that im2col fills from it; every element of im is written. */
int tt_col2im(int dtype, const void* col, void* im, int64_t N, int C, int H, int W, int kh, int kw, int pad_h,
              int pad_w, int stride_h, int stride_w, void* stream);

/* Max pooling over `planes` images [H][W] (batch x channels): out and mask
 * [planes][OH][OW] (OH, OW as for im2col); the window is clipped to the
 * image, the first largest entry in row-major order wins, mask holds its index
 * y * W + x as a float (-1, out -FLT_MAX, for a window with no image element):
 * the reference's MaxPoolingForward (src/Layers.cu:254-286, kernel
 * src/Layers_kernels.cu:109-153). */
int tt_maxpool_f32(const float* in, float* out, float* mask, int64_t planes, int H, int W, int kh, int kw, int pad_h,
                   int pad_w, int stride_h, int stride_w, void* stream);
/* grad_in [planes][H][W] = the sum of grad_out over the windows whose mask
 * points at each element (MaxPoolingBackward, src/Layers.cu:288-322, assigns
 * instead: equal for non-overlapping windows); every element is written. */
int tt_maxpool_backward_f32(const float* grad_out, const float* mask, float* grad_in, int64_t planes, int H, int W,
                            int kh, int kw, int pad_h, int pad_w, int stride_h, int stride_w, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TT_ATTN_H */
