"""CPU oracle for TinyTensor scaled dot-product attention (fwd, bwd, decode),
the row softmax of ``myLayer.SoftmaxForward`` and the ``cudaGemm`` contract.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg, never by the product package.

The reference (csxq0605/pku-aiprogramming, "TinyTensor") has no attention
operator.  Its attention op is the composition of its own autodiff ops:

  O = softmax((Q @ K.T) * s + M) @ V

built from ``MatMul`` (Task3/Tinytensor/optimizer/operators.py:416-419),
``Transpose`` (operators.py:323-336, default swaps the last two axes),
``MulScalar`` (operators.py:234-239), ``EWiseAdd`` with a constant -inf
upper-triangle mask (operators.py:194-196), and the stable softmax formula
max-shift -> exp -> sum -> divide (operators.py:611-612, and the GPU order of
``SoftmaxForward``, Task3/Tinytensor/src/Layers.cu:324-349), then ``@ V``.
The backward is ``O.backward(dO)`` (operators.py:115-119 ->
autodiff.py:33-61) through the gradient rules of those ops.

Two restatements live here:

* ``attn_fwd_f64`` / ``attn_bwd_f64`` / ``attn_decode_f64`` -- the closed form
  in float64.  This is the ground truth every kernel is compared against.
* ``composition_fwd_f32`` / ``composition_bwd_f32`` -- the reference's own op
  sequence in float32 numpy, gradient rule by gradient rule, materialising S
  and P over the full L x L even when causal (the reference never skips
  masked work).  This is the timed CPU baseline.

Pinning (see tests/test_oracle.py): brute-force loops at c1 size, torch CPU
``scaled_dot_product_attention`` + autograd in float64, central finite
differences, closed forms (causal row 0, constant scores, LSE of Q=0,
constant-V backward), invariants (row sums, shift invariance, sum of dS, causal
independence of future rows, decode split-merge) and committed golden vectors
written by torch, not by this file.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import numpy as np

LOG2E = 1.4426950408889634

# ---------------------------------------------------------------------------
# bfloat16 helpers (numpy has no bf16 dtype).  Round-to-nearest-even on the
# float32 bit pattern; NaN is kept quiet.
# ---------------------------------------------------------------------------


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    lsb = (u >> 16) & 1
    r = ((u.astype(np.uint64) + 0x7FFF + lsb) >> 16).astype(np.uint16)
    if nan.any():
        r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> float32 (exact)."""
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 values rounded to the nearest bf16, returned as float32."""
    return bf16_to_f32(bf16_bits(x))


# ---------------------------------------------------------------------------
# Benchmark configurations and seeded inputs
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class AttnConfig:
    cid: int
    B: int
    H: int
    Lq: int
    Lk: int
    d: int
    dtype: str          # "f32" or "bf16"
    causal: bool
    backward: bool
    qkv_scale: float = 1.0

    @property
    def scale(self) -> float:
        return float(np.float32(1.0 / math.sqrt(self.d)))

    def fwd_flops(self) -> float:
        f = 4.0 * self.B * self.H * self.Lq * self.Lk * self.d
        return f / 2 if self.causal else f

    def bwd_flops(self) -> float:
        f = 8.0 * self.B * self.H * self.Lq * self.Lk * self.d
        return f / 2 if self.causal else f


CONFIGS: Dict[int, AttnConfig] = {
    1: AttnConfig(1, 1, 1, 64, 64, 32, "f32", False, False),
    2: AttnConfig(2, 8, 8, 256, 256, 64, "f32", False, True),
    3: AttnConfig(3, 16, 16, 1024, 1024, 64, "bf16", True, True, 0.5),
    4: AttnConfig(4, 64, 32, 1, 8192, 128, "bf16", False, False),
    5: AttnConfig(5, 4, 32, 4096, 4096, 128, "bf16", True, True),
}


def seeded_inputs(cfg: AttnConfig, with_kv: bool = True) -> Dict[str, np.ndarray]:
    """Inputs of config ``cfg``: ``np.random.default_rng(cid)``, drawn in the
    order Q, K, V, dO with ``standard_normal(float32)``.  Q/K/V are scaled by
    ``qkv_scale``; bf16 configs round every tensor with RNE.  Returns float32
    arrays holding exactly the values the kernel sees."""
    rng = np.random.default_rng(cfg.cid)
    qs = (cfg.B, cfg.H, cfg.Lq, cfg.d)
    ks = (cfg.B, cfg.H, cfg.Lk, cfg.d)
    out = {}
    out["q"] = rng.standard_normal(qs, dtype=np.float32)
    if with_kv:
        out["k"] = rng.standard_normal(ks, dtype=np.float32)
        out["v"] = rng.standard_normal(ks, dtype=np.float32)
    if cfg.backward:
        out["do"] = rng.standard_normal(qs, dtype=np.float32)
    if cfg.qkv_scale != 1.0:
        for n in ("q", "k", "v"):
            if n in out:
                out[n] *= np.float32(cfg.qkv_scale)
    if cfg.dtype == "bf16":
        for n in out:
            out[n] = bf16_round(out[n])
    return out


# ---------------------------------------------------------------------------
# float64 ground truth
# ---------------------------------------------------------------------------


def _causal_mask(Lq: int, Lk: int) -> np.ndarray:
    """True where masked: key j > query i (strict upper triangle, top-left
    aligned), the constant -inf tensor the reference adds with EWiseAdd."""
    return np.triu(np.ones((Lq, Lk), dtype=bool), k=1)


def attn_fwd_f64(q, k, v, scale: float, causal: bool) -> Tuple[np.ndarray, np.ndarray]:
    """O = softmax(s * Q K^T + M) V and LSE_i = m_i + ln sum_j exp(S_ij - m_i).

    Follows operators.py:163-164 (Q @ K^T), :234-239 (x s), :194-196 (+ mask),
    :611-612 (max-shift, exp, sum, divide), then @ V.  float64 throughout.
    Shapes [..., L, d]; returns O [..., Lq, d] and LSE [..., Lq]."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    s = np.matmul(q, np.swapaxes(k, -1, -2)) * float(scale)
    if causal:
        s = np.where(_causal_mask(s.shape[-2], s.shape[-1]), -np.inf, s)
    m = np.max(s, axis=-1, keepdims=True)
    e = np.exp(s - m)
    z = np.sum(e, axis=-1, keepdims=True)
    p = e / z
    o = np.matmul(p, v)
    lse = (m + np.log(z))[..., 0]
    return o, lse


def attn_probs_f64(q, k, scale: float, causal: bool) -> np.ndarray:
    """P = softmax(s Q K^T + M) in float64 (used by invariant tests)."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    s = np.matmul(q, np.swapaxes(k, -1, -2)) * float(scale)
    if causal:
        s = np.where(_causal_mask(s.shape[-2], s.shape[-1]), -np.inf, s)
    m = np.max(s, axis=-1, keepdims=True)
    e = np.exp(s - m)
    return e / np.sum(e, axis=-1, keepdims=True)


def attn_bwd_f64(q, k, v, do, scale: float, causal: bool):
    """dQ, dK, dV of O = softmax(s Q K^T + M) V for upstream grad dO, float64.

    The reference reaches these through MatMul.gradient (operators.py:421-429),
    Transpose.gradient (:338-340), MulScalar.gradient (:241-242),
    EWiseDiv.gradient (:296-298), BroadcastTo/Summation gradients (:373-380,
    :400-408) and Exp.gradient (:469-470).  Closed form of that chain:
    dV = P^T dO; dP = dO V^T; D_i = sum_j P_ij dP_ij (= rowsum(dO o O));
    dS = P o (dP - D); dQ = s dS K; dK = s dS^T Q."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    do = np.asarray(do, np.float64)
    p = attn_probs_f64(q, k, scale, causal)
    dv = np.matmul(np.swapaxes(p, -1, -2), do)
    dp = np.matmul(do, np.swapaxes(v, -1, -2))
    dsum = np.sum(p * dp, axis=-1, keepdims=True)
    ds = p * (dp - dsum)
    dq = np.matmul(ds, k) * float(scale)
    dk = np.matmul(np.swapaxes(ds, -1, -2), q) * float(scale)
    return dq, dk, dv


def attn_decode_f64(q, k, v, scale: float) -> Tuple[np.ndarray, np.ndarray]:
    """Single-query decode: the forward with Lq = 1 and no mask.
    q [..., 1, d], K/V [..., Lkv, d] -> o [..., 1, d], lse [..., 1]."""
    return attn_fwd_f64(q, k, v, scale, False)


def decode_split_merge_f64(q, k, v, scale: float, splits: int):
    """Decode computed over ``splits`` contiguous Lkv chunks, each giving a
    partial (o_c, lse_c), merged by LSE rescaling:
    lse = log sum_c exp(lse_c); o = sum_c exp(lse_c - lse) o_c.
    Equal to ``attn_decode_f64`` for any split (invariance checked in tests)."""
    Lk = k.shape[-2]
    bounds = np.linspace(0, Lk, splits + 1).astype(int)
    parts = []
    for c in range(splits):
        a, b = bounds[c], bounds[c + 1]
        if b > a:
            parts.append(attn_fwd_f64(q, k[..., a:b, :], v[..., a:b, :], scale, False))
    lses = np.stack([p[1] for p in parts])
    mx = np.max(lses, axis=0)
    w = np.exp(lses - mx)
    lse = mx + np.log(np.sum(w, axis=0))
    o = sum(np.exp(p[1] - lse)[..., None] * p[0] for p in parts)
    return o, lse


# ---------------------------------------------------------------------------
# The reference's op sequence in float32 (timed CPU baseline)
# ---------------------------------------------------------------------------


def composition_fwd_f32(q, k, v, scale: float, causal: bool, keep: bool = False):
    """Forward in the reference's op order, float32 numpy:
    Kt = Transpose(K)               operators.py:323-336
    S0 = MatMul(Q, Kt)              operators.py:416-419
    S1 = MulScalar(s)(S0)           operators.py:234-239
    S2 = EWiseAdd(S1, mask)         operators.py:194-196 (causal only)
    S3 = S2 - rowmax (a constant)   operators.py:611
    E  = Exp(S3)                    operators.py:464-466
    Z  = Summation((3,))(E)         operators.py:388-397
    Zb = BroadcastTo(Reshape(Z))    operators.py:348-353, 366-371
    P  = EWiseDiv(E, Zb)            operators.py:289-293
    O  = MatMul(P, V)
    Returns O (and the saved intermediates when ``keep``)."""
    q = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    v = np.asarray(v, np.float32)
    s = np.float32(scale)
    kt = np.swapaxes(k, -1, -2)
    s0 = np.matmul(q, kt)
    s1 = s0 * s
    if causal:
        mask = np.where(_causal_mask(s1.shape[-2], s1.shape[-1]), np.float32(-np.inf), np.float32(0))
        s2 = s1 + mask
    else:
        s2 = s1
    mx = np.max(s2, axis=-1, keepdims=True)
    s3 = s2 - mx
    e = np.exp(s3)
    z = np.sum(e, axis=-1)
    zb = np.broadcast_to(np.reshape(z, z.shape + (1,)), e.shape)
    p = e / zb
    o = np.matmul(p, v)
    if keep:
        return o, dict(s3=s3, e=e, zb=zb, p=p)
    return o


def composition_bwd_f32(q, k, v, do, scale: float, causal: bool):
    """Backward of ``composition_fwd_f32`` by the reference's own gradient
    rules, in the order compute_gradient_of_variables (autodiff.py:33-61)
    visits them, float32:
    MatMul(P, V):   dP = dO @ V^T, dV = P^T @ dO         operators.py:421-429
    EWiseDiv(E,Zb): dE1 = dP / Zb; dZb = (-dP) * E / Zb**2  operators.py:296-298
    BroadcastTo:    dZr = Reshape(Summation(dZb, (3,)))   operators.py:373-380
    Summation:      dE2 = BroadcastTo(Reshape(dZ))        operators.py:400-408
    E's grads summed in list order: dE = dE1 + dE2        autodiff.py:49-53
    Exp:            dS3 = dE * exp(S3)                    operators.py:469-470
    EWiseAdd:       pass-through                          operators.py:198-199
    MulScalar:      dS0 = dS1 * s                         operators.py:241-242
    MatMul(Q, Kt):  dQ = dS0 @ K, dKt = Q^T @ dS0         operators.py:421-429
    Transpose:      dK = Transpose(dKt)                   operators.py:338-340
    Returns dQ, dK, dV."""
    q = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    v = np.asarray(v, np.float32)
    do = np.asarray(do, np.float32)
    s = np.float32(scale)
    _, sv = composition_fwd_f32(q, k, v, scale, causal, keep=True)
    p, e, zb, s3 = sv["p"], sv["e"], sv["zb"], sv["s3"]
    dp = np.matmul(do, np.swapaxes(v, -1, -2))
    dv = np.matmul(np.swapaxes(p, -1, -2), do)
    de1 = dp / zb
    dzb = (-dp) * e / (zb ** 2)
    dz = np.sum(dzb, axis=-1)
    de2 = np.broadcast_to(np.reshape(dz, dz.shape + (1,)), e.shape)
    de = de1 + de2
    ds3 = de * np.exp(s3)
    ds0 = ds3 * s
    dq = np.matmul(ds0, k)
    dkt = np.matmul(np.swapaxes(q, -1, -2), ds0)
    dk = np.swapaxes(dkt, -1, -2)
    return dq, dk, dv


# ---------------------------------------------------------------------------
# Row softmax: SoftmaxForward (Task3/Tinytensor/src/Layers.cu:324-349)
# ---------------------------------------------------------------------------


def softmax_rows_f64(x) -> np.ndarray:
    """Closed form over the last axis in float64: exp(x - max) / sum exp(x - max)."""
    x = np.asarray(x, np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        e = np.exp(x - np.max(x, axis=-1, keepdims=True))
        return e / np.sum(e, axis=-1, keepdims=True)


def softmax_rows_ref_f32(x) -> np.ndarray:
    """The reference's GPU op order in float32 (Layers.cu:330-348): per-row max
    (cudaChannelMax, Layers_kernels.cu:190-205), x - max (cudaChannelSub,
    :222-235), exp (cudaChannelExp, :250-259), per-row sum (cudaChannelSum,
    :206-221), divide (cudaChannelDiv, :236-249); also the CPU formula of
    Softmaxloss.compute (optimizer/operators.py:611-612)."""
    x = np.asarray(x, np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        m = np.max(x, axis=-1, keepdims=True)
        e = np.exp(x - m).astype(np.float32)
        return (e / np.sum(e, axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)


# ---------------------------------------------------------------------------
# GEMM: the cudaGemm contract (Task3/Tinytensor/src/Layers_kernels.cu:10-30)
# ---------------------------------------------------------------------------


def gemm_f64(transa: bool, transb: bool, alpha: float, A, B, beta: float, C=None) -> np.ndarray:
    """alpha op(A) @ op(B) + beta C in float64, row-major.  op(A) = A.T when
    transa (A stored k x m), op(B) = B.T when transb (B stored n x k); the
    reference reaches the same product by calling cublasSgemm on the
    column-major views with the operands swapped (Layers_kernels.cu:22-27).
    beta = 0 ignores C (it may hold anything)."""
    a = np.asarray(A, np.float64)
    b = np.asarray(B, np.float64)
    a = a.T if transa else a
    b = b.T if transb else b
    out = alpha * (a @ b)
    if beta != 0.0:
        out = out + beta * np.asarray(C, np.float64)
    return out


# ---------------------------------------------------------------------------
# Error metric
# ---------------------------------------------------------------------------


def max_rel_err(x, ref) -> float:
    """Normwise max relative error: max|x - ref| / max|ref|."""
    x = np.asarray(x, np.float64)
    ref = np.asarray(ref, np.float64)
    if ref.size == 0:
        return 0.0
    if not np.array_equal(np.isfinite(x), np.isfinite(ref)):
        return math.inf
    fin = np.isfinite(ref)
    if not np.array_equal(x[~fin], ref[~fin]):
        return math.inf
    x, ref = x[fin], ref[fin]
    if ref.size == 0:
        return 0.0
    den = float(np.max(np.abs(ref)))
    num = float(np.max(np.abs(x - ref)))
    if den == 0.0:
        return num
    return num / den


def elem_rel_err(x, ref) -> float:
    """Elementwise max |x - ref| / (|ref| + 1e-6 max|ref|), for diagnosis."""
    x = np.asarray(x, np.float64)
    ref = np.asarray(ref, np.float64)
    if ref.size == 0:
        return 0.0
    floor = 1e-6 * float(np.max(np.abs(ref)))
    return float(np.max(np.abs(x - ref) / (np.abs(ref) + floor + 1e-300)))


# Tolerances stated by the north star: fp32 <= 1e-4, bf16 (fp32 accumulation) <= 2e-2.
TOL = {"f32": 1e-4, "bf16": 2e-2}
