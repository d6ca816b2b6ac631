"""GPU test of the allocation-free backward entry point
(tt_attn_bwd_bf16_noalloc) through the C-ABI: calls in a row, each with a
smaller input than the one before, each against tt_attn_bwd_bf16 on the
same inputs (the same kernels, so the results must agree bit for bit) and
against the float64 oracle, with the library allocator's statistics
unchanged by the calls; sizes beyond the static scratch are refused before
any launch.
"""
import ctypes as C
import math

import numpy as np
import pytest

from oracle import attn_oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def capi():
    import tt_capi

    assert tt_capi.lib().device_count() >= 1
    tt_capi.lib().call("tt_init", 0)
    return tt_capi


def _inputs(capi, seed, B, H, L, d):
    rng = np.random.default_rng(seed)
    x = {n: orc.bf16_round(rng.standard_normal((B, H, L, d), dtype=np.float32)) for n in ("q", "k", "v", "do")}
    return x, {n: capi.DeviceBuffer.from_numpy(a, "bf16") for n, a in x.items()}


def _bwd(capi, name, b, o, lse, scale, causal):
    B, H, L, d = b["q"].shape
    g = [capi.DeviceBuffer(b["q"].shape, "bf16") for _ in range(3)]
    capi.lib().call(name, b["q"].ptr, b["k"].ptr, b["v"].ptr, o.ptr, lse.ptr, b["do"].ptr, g[0].ptr, g[1].ptr,
                    g[2].ptr, B, H, L, L, d, C.c_float(scale), int(causal), None)
    return g


def _stats(capi):
    used, cached = C.c_size_t(), C.c_size_t()
    capi.lib().call("tt_mem_stats", C.byref(used), C.byref(cached))
    return used.value, cached.value


@pytest.mark.parametrize("order", ["large_then_small"])
def test_noalloc_backward_matches_the_allocating_entry_point(capi, order):
    # each call smaller than the one before (B*H*L rows: 4096, 2304, 1200,
    # 600, 260), covering d = 128 and d = 64 (the dQ kernel writes the rows
    # into the static scratch) and d = 32 (a separate row pre-pass kernel
    # writes them), causal and not
    cases = [(11, 2, 4, 512, 128, True), (13, 2, 3, 384, 64, True), (14, 1, 4, 300, 32, True),
             (12, 1, 3, 200, 64, False), (15, 1, 2, 130, 32, False)]
    for seed, B, H, L, d, causal in cases:
        print(f"noalloc bwd B={B} H={H} L={L} d={d} causal={causal}", flush=True)
        scale = float(np.float32(1 / math.sqrt(d)))
        x, b = _inputs(capi, seed, B, H, L, d)
        o = capi.DeviceBuffer((B, H, L, d), "bf16")
        lse = capi.DeviceBuffer((B, H, L), "f32")
        capi.attn_fwd(b["q"], b["k"], b["v"], o, lse, scale, causal)
        ref = _bwd(capi, "tt_attn_bwd_bf16", b, o, lse, scale, causal)
        outs = [capi.DeviceBuffer((B, H, L, d), "bf16") for _ in range(3)]
        capi.lib().sync()
        before = _stats(capi)
        capi.lib().call("tt_attn_bwd_bf16_noalloc", b["q"].ptr, b["k"].ptr, b["v"].ptr, o.ptr, lse.ptr, b["do"].ptr,
                        outs[0].ptr, outs[1].ptr, outs[2].ptr, B, H, L, L, d, C.c_float(scale), int(causal), None)
        capi.lib().sync()
        assert _stats(capi) == before  # nothing allocated or freed by the call
        for n, got, want in zip(("dQ", "dK", "dV"), outs, ref):
            np.testing.assert_array_equal(got.download_bytes(), want.download_bytes(), err_msg=n)
        rq, rk, rv = orc.attn_bwd_f64(x["q"], x["k"], x["v"], x["do"], scale, causal)
        for n, got, r in zip(("dQ", "dK", "dV"), outs, (rq, rk, rv)):
            assert orc.max_rel_err(got.download(), r) <= orc.TOL["bf16"], n


def test_noalloc_backward_refuses_sizes_beyond_the_scratch(capi):
    L = capi.lib()
    p = C.c_void_p(16)  # never dereferenced: the size check comes first
    rc = L.lib.tt_attn_bwd_bf16_noalloc(p, p, p, p, p, p, p, p, p, 64, 32, 1025, 1025, 64, C.c_float(0.125), 1, None)
    assert rc == capi.TT_ERR_ARG and "static scratch maximum" in L.last_error()
