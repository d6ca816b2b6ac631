"""GPU tests of concurrent use and failure handling of the C-ABI:

* two host threads, each with its own caller stream (default priority),
  running attention backward calls of different shapes at the same time:
  every result matches the float64 oracle (the per-stream workspaces keep
  their -D / LSE buffers apart), also with two persistent d = 128 dK/dV
  launches sharing the CUs;
* one stream shared by two threads: the workspace lease keeps each call's
  launches together, so both threads' results stay correct;
* allocation-failure injection (TT_FAIL_ALLOC_AFTER) in a child process:
  tt_malloc and the backward's workspace report TT_ERR_NOMEM with a message,
  and the library keeps working for calls that need no new memory.
"""
import math
import os
import subprocess
import sys
import threading

import numpy as np
import pytest

from oracle import attn_oracle as orc

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def capi():
    import tt_capi

    assert tt_capi.lib().device_count() >= 1
    return tt_capi


def _case(seed, B, H, L, d, causal):
    rng = np.random.default_rng(seed)
    x = {n: orc.bf16_round(rng.standard_normal((B, H, L, d), dtype=np.float32)) for n in ("q", "k", "v", "do")}
    scale = float(np.float32(1 / math.sqrt(d)))
    o, lse = orc.attn_fwd_f64(x["q"], x["k"], x["v"], scale, causal)
    ref = orc.attn_bwd_f64(x["q"], x["k"], x["v"], x["do"], scale, causal)
    return x, scale, o, ref


def _run_on(capi, stream, x, scale, causal):
    """Forward + backward on `stream` (a handle, or None); returns dQ, dK, dV."""
    shp = x["q"].shape
    b = {n: capi.DeviceBuffer.from_numpy(a, "bf16") for n, a in x.items()}
    o = capi.DeviceBuffer(shp, "bf16")
    lse = capi.DeviceBuffer(shp[:3], "f32")
    g = [capi.DeviceBuffer(shp, "bf16") for _ in range(3)]
    capi.attn_fwd(b["q"], b["k"], b["v"], o, lse, scale, causal, stream=stream)
    capi.attn_bwd(b["q"], b["k"], b["v"], o, lse, b["do"], *g, scale, causal, stream=stream)
    capi.lib().call("tt_stream_sync", stream)
    return [t.download() for t in g]


def _threads(capi, streams, cases, reps):
    errors = []

    def work(i):
        try:
            x, scale, _, ref = cases[i]
            for _ in range(reps):
                got = _run_on(capi, streams[i], x, scale, True)
                for n, a, r in zip(("dQ", "dK", "dV"), got, ref):
                    e = orc.max_rel_err(a, r)
                    if e > orc.TOL["bf16"]:
                        errors.append(f"thread {i} {n}: {e:.3e}")
        except Exception as exc:  # surfaced below
            errors.append(f"thread {i}: {exc!r}")

    th = [threading.Thread(target=work, args=(i,)) for i in range(len(cases))]
    for t in th:
        t.start()
    for t in th:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in th), "a worker thread did not finish"
    assert not errors, errors


def test_two_threads_two_streams_backward(capi):
    cases = [_case(1, 2, 4, 384, 128, True), _case(2, 1, 6, 256, 64, True)]
    streams = [capi.Stream(), capi.Stream()]
    _say("two threads, two streams: bf16 causal bwd [2,4,384,128] and [1,6,256,64], 4 reps each")
    try:
        _threads(capi, [s.handle for s in streams], cases, reps=4)
    finally:
        for s in streams:
            s.destroy()


def test_two_threads_two_streams_persistent_d128(capi):
    # both calls run the persistent d = 128 dK/dV launch (one workgroup per CU
    # at most): launches on the two streams share the CUs and must not wait
    # for each other
    cases = [_case(5, 2, 4, 384, 128, True), _case(6, 1, 8, 640, 128, True)]
    streams = [capi.Stream(), capi.Stream()]
    _say("two threads, two streams: bf16 causal bwd [2,4,384,128] and [1,8,640,128], 4 reps each")
    try:
        _threads(capi, [s.handle for s in streams], cases, reps=4)
    finally:
        for s in streams:
            s.destroy()


def test_two_threads_one_shared_stream(capi):
    cases = [_case(3, 1, 4, 320, 128, True), _case(4, 2, 2, 192, 64, True)]
    s = capi.Stream()
    _say("two threads, one stream: bf16 causal bwd [1,4,320,128] and [2,2,192,64], 4 reps each")
    try:
        _threads(capi, [s.handle, s.handle], cases, reps=4)
    finally:
        s.destroy()


def test_two_streams_fp32_split_forward(capi):
    """The fp32 forward of a small problem splits its keys and merges the
    partials through a per-stream workspace: two threads, two streams,
    different shapes, every result against the oracle (fp32 bar)."""
    shapes = [(1, 3, 200, 64, False), (2, 2, 130, 128, True)]
    streams = [capi.Stream(), capi.Stream()]
    errors = []

    def work(i):
        try:
            B, H, L, d, causal = shapes[i]
            rng = np.random.default_rng(40 + i)
            x = {n: rng.standard_normal((B, H, L, d), dtype=np.float32) for n in ("q", "k", "v")}
            scale = float(np.float32(1 / math.sqrt(d)))
            o_ref, l_ref = orc.attn_fwd_f64(x["q"], x["k"], x["v"], scale, causal)
            b = {n: capi.DeviceBuffer.from_numpy(a, "f32") for n, a in x.items()}
            for _ in range(4):
                o = capi.DeviceBuffer((B, H, L, d), "f32")
                lse = capi.DeviceBuffer((B, H, L), "f32")
                capi.attn_fwd(b["q"], b["k"], b["v"], o, lse, scale, causal, stream=streams[i].handle)
                capi.lib().call("tt_stream_sync", streams[i].handle)
                for n, a, r in (("O", o.download(), o_ref), ("LSE", lse.download(), l_ref)):
                    e = orc.max_rel_err(a, r)
                    if e > orc.TOL["f32"]:
                        errors.append(f"thread {i} {n}: {e:.3e}")
        except Exception as exc:  # surfaced below
            errors.append(f"thread {i}: {exc!r}")

    _say("two threads, two streams: fp32 split forward [1,3,200,64] and causal [2,2,130,128], 4 reps each")
    try:
        th = [threading.Thread(target=work, args=(i,)) for i in range(2)]
        for t in th:
            t.start()
        for t in th:
            t.join(timeout=120)
        assert not any(t.is_alive() for t in th), "a worker thread did not finish"
        assert not errors, errors
    finally:
        for st in streams:
            st.destroy()


def test_library_stream_cannot_be_destroyed(capi):
    L = capi.lib()
    rc = L.lib.tt_stream_destroy(L.lib.tt_stream())
    assert rc == capi.TT_ERR_ARG and "library stream" in L.last_error()


CHILD = r"""
import ctypes as C, sys
sys.path.insert(0, sys.argv[1])
import tt_capi as T
L = T.lib()
ok = [T.DeviceBuffer((4, 256, 64), "bf16") for _ in range(8)]     # allocations 0..7 succeed
p = C.c_void_p()
rc = L.lib.tt_malloc(C.byref(p), 1 << 20)                          # allocation 8: refused
assert rc == T.TT_ERR_NOMEM, rc
assert "failure injection" in L.last_error(), L.last_error()
q, k, v, do, o, gq, gk, gv = ok
for b in ok:
    b.zero()
# the backward needs a workspace buffer (a new allocation): refused cleanly
# (the fp32 LSE rows, all zero, are read from the start of o's buffer)
rc = L.lib.tt_attn_bwd_bf16(q.ptr, k.ptr, v.ptr, o.ptr, o.ptr, do.ptr, gq.ptr, gk.ptr, gv.ptr,
                            1, 4, 256, 256, 64, C.c_float(0.125), 1, None)
assert rc == T.TT_ERR_NOMEM, (rc, L.last_error())
# a forward needs no allocation: still works after the failures
rc = L.lib.tt_attn_fwd_bf16(q.ptr, k.ptr, v.ptr, o.ptr, None, 1, 4, 256, 256, 64, C.c_float(0.125), 1, None)
assert rc == T.TT_OK, L.last_error()
L.sync()
print("CHILD_OK")
"""


def test_allocation_failure_injection(capi):
    env = dict(os.environ, TT_FAIL_ALLOC_AFTER="8")
    r = subprocess.run([sys.executable, "-c", CHILD, os.path.join(ROOT, "pku-aiprogramming_amd")],
                       capture_output=True, text=True, timeout=120, env=env)
    _say(r.stdout[-500:] + r.stderr[-2000:])
    assert r.returncode == 0 and "CHILD_OK" in r.stdout


def test_read_probe_reads_and_stores_nothing(capi):
    """The bench's read-rate probe: a ragged size (not a whole number of
    256 KiB runs) runs without error and leaves its sink alone (zero data
    never sums to the sentinel)."""
    L = capi.lib()
    buf = capi.DeviceBuffer(((1 << 18) + 12,), "f32")  # 1 MiB + 48 bytes
    buf.zero()
    sink = capi.DeviceBuffer.from_numpy(np.array([7.0], dtype=np.float32), "f32")
    L.check(L.lib.tt_read_probe(buf.ptr, buf.nbytes, sink.ptr, None), "tt_read_probe")
    L.sync()
    assert sink.download()[0] == 7.0
