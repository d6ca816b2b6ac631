"""GPU parity tests of the MFMA GEMM (``tt_gemm_f32`` / ``tt_gemm_bf16``, the
cudaGemm contract of src/Layers_kernels.cu:10-30) against the float64 oracle
(``oracle.attn_oracle.gemm_f64``) on the exact (for bf16: bf16-rounded)
inputs.

Bar (normwise max|C - ref| / max|ref|): fp32 <= 1e-5 (fp32 products on the
fp32 MFMA, fp32 sums over k <= 4096 terms); bf16 <= 8e-3 (C is rounded to
bf16, half an ulp = 2^-9, plus fp32 sums).  Shapes cover every transpose
combination, exact tiles and ragged edges in m, n and k, vectors, k = 0,
beta != 0 (C read) and leading dimensions that rule out 16-byte loads.
"""
import sys

import numpy as np
import pytest

from oracle import attn_oracle as orc

pytestmark = pytest.mark.gpu

TOL = {"f32": 1e-5, "bf16": 8e-3}


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def capi():
    import tt_capi

    assert tt_capi.lib().device_count() >= 1, "no HIP device visible"
    return tt_capi


def _run(capi, dt, ta, tb, m, n, k, alpha=1.0, beta=0.0, seed=0):
    rng = np.random.default_rng(seed + 7 * m + 13 * n + 17 * k + 2 * ta + tb)
    A = rng.standard_normal((k, m) if ta else (m, k)).astype(np.float32)
    B = rng.standard_normal((n, k) if tb else (k, n)).astype(np.float32)
    C = rng.standard_normal((m, n)).astype(np.float32)
    if dt == "bf16":
        A, B, C = orc.bf16_round(A), orc.bf16_round(B), orc.bf16_round(C)
    dA = capi.DeviceBuffer.from_numpy(A, dt)
    dB = capi.DeviceBuffer.from_numpy(B, dt)
    dC = capi.DeviceBuffer.from_numpy(C, dt)
    capi.gemm(ta, tb, m, n, k, alpha, dA, dB, beta, dC)
    capi.lib().sync()
    out = dC.download().reshape(m, n)
    ref = orc.gemm_f64(ta, tb, alpha, A, B, beta, C)
    err = orc.max_rel_err(out, ref)
    _say(f"  gemm {dt} ta={int(ta)} tb={int(tb)} m={m} n={n} k={k} alpha={alpha} beta={beta}: max-rel-err {err:.3e}")
    assert err <= TOL[dt], err
    return out


SHAPES = [
    (1, 1, 1), (7, 5, 3), (128, 128, 64), (256, 128, 128), (129, 130, 65), (300, 257, 1000), (1000, 1, 37),
    (2, 3000, 17), (64, 64, 4096), (1024, 1024, 1024),
    # k a multiple of 32 (the bf16 direct-to-LDS kernel): full 128 x 256 tiles,
    # then ragged m / n (multiples of 8, so every transpose combination runs it)
    (512, 768, 96), (128, 256, 32), (256, 512, 2048),
    (136, 264, 96), (1000, 8, 64), (8, 1000, 32), (520, 776, 2048),
]


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
@pytest.mark.parametrize("shape", SHAPES, ids=[str(s) for s in SHAPES])
def test_gemm_shapes(capi, dt, ta, tb, shape):
    m, n, k = shape
    _run(capi, dt, ta, tb, m, n, k)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_gemm_alpha_beta_and_k0(capi, dt):
    _run(capi, dt, False, False, 200, 150, 96, alpha=0.5, beta=1.5)
    _run(capi, dt, True, True, 130, 70, 40, alpha=-2.0, beta=1.0)
    _run(capi, dt, False, True, 33, 65, 0, alpha=1.0, beta=3.0)   # k = 0: C = beta C
    _run(capi, dt, True, False, 256, 512, 64, alpha=0.75, beta=-0.5)   # full tiles, C read


def test_gemm_beta_zero_ignores_c(capi):
    """beta = 0 never reads C: a NaN-filled C comes back finite."""
    A = np.ones((64, 32), np.float32)
    B = np.ones((32, 48), np.float32)
    dA, dB = capi.DeviceBuffer.from_numpy(A, "f32"), capi.DeviceBuffer.from_numpy(B, "f32")
    dC = capi.DeviceBuffer.from_numpy(np.full((64, 48), np.nan, np.float32), "f32")
    capi.gemm(False, False, 64, 48, 32, 1.0, dA, dB, 0.0, dC)
    capi.lib().sync()
    np.testing.assert_array_equal(dC.download().reshape(64, 48), np.full((64, 48), 32.0, np.float32))


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_gemm_fc_layer_call_pattern(capi, dt):
    """The three GEMMs of FcForward / FcBackward (src/Layers.cu:26, 65-66):
    out = in W; d_in = d_out W^T; dW = in^T d_out, at an MNIST-like shape."""
    batch, fin, fout = 100, 784, 256
    _run(capi, dt, False, False, batch, fout, fin)          # out = in @ W
    _run(capi, dt, False, True, batch, fin, fout)           # d_in = d_out @ W^T
    _run(capi, dt, True, False, fin, fout, batch)           # dW = in^T @ d_out
