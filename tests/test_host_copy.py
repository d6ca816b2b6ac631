"""CPU tests of the staged transfers' host loops (csrc/host_copy.cpp): the
byte copy and the float32 <-> bf16 conversions with non-temporal stores,
compiled here with a small extern "C" shim and compared with numpy at every
destination / source alignment, lengths around the 64-byte steps, and the
special float values.  Bar: bit-exact; bf16 equals numpy's round to nearest
even (the oracle's bf16 rounding) on non-NaN values, NaNs stay quiet NaNs of
the same sign.
"""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

from oracle import attn_oracle as orc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "pku-aiprogramming_amd", "csrc")

SHIM = r"""
#include "host_copy.h"
extern "C" {
void hc_copy(void* d, const void* s, size_t n) { tt::copy_stream(d, s, n); }
void hc_f2b(void* d, const void* s, size_t n) { tt::f32_to_bf16_stream((uint16_t*)d, (const float*)s, n); }
void hc_b2f(void* d, const void* s, size_t n) { tt::bf16_to_f32_stream((float*)d, (const uint16_t*)s, n); }
}
"""


@pytest.fixture(scope="module")
def hc(tmp_path_factory):
    d = tmp_path_factory.mktemp("hc")
    shim = d / "shim.cpp"
    shim.write_text(SHIM)
    so = d / "libhc.so"
    subprocess.run(["g++", "-O2", "-fPIC", "-shared", "-std=c++17", "-I", CSRC, str(shim),
                    os.path.join(CSRC, "host_copy.cpp"), "-o", str(so)], check=True)
    lib = C.CDLL(str(so))
    for f in ("hc_copy", "hc_f2b", "hc_b2f"):
        getattr(lib, f).argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
        getattr(lib, f).restype = None
    return lib


LENGTHS = [0, 1, 2, 7, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 1000, 4099]


@pytest.mark.parametrize("n", LENGTHS)
def test_copy_every_alignment(hc, n):
    rng = np.random.default_rng(n)
    src = rng.integers(0, 256, n + 64, dtype=np.uint8)
    for doff in range(16):
        for soff in (0, 1, 3, 8):
            dst = np.full(n + 64, 0xAA, np.uint8)
            hc.hc_copy(dst.ctypes.data + doff, src.ctypes.data + soff, n)
            np.testing.assert_array_equal(dst[doff:doff + n], src[soff:soff + n])
            assert (dst[:doff] == 0xAA).all() and (dst[doff + n:] == 0xAA).all()


def _special():
    bits = np.array([0, 0x80000000, 1, 0x807FFFFF, 0x8000, 0x18000, 0x28000, 0x3F808000, 0x3F818000,
                     0x3F80FFFF, 0x3F807FFF, 0x7F7FFFFF, 0xFF7FFFFF, 0x7F7F7FFF, 0x7F800000, 0xFF800000,
                     0x7F800001, 0x7FC00000, 0xFFFFFFFF, 0x7FBFFFFF, 0xFFFF8001, 0xFFFF8000], np.uint32)
    return bits.view(np.float32)


@pytest.mark.parametrize("n", LENGTHS)
def test_f32_to_bf16_every_alignment(hc, n):
    rng = np.random.default_rng(100 + n)
    x = (rng.standard_normal(n + 8) * 1000).astype(np.float32)
    sp = _special()
    x[: min(n, sp.size)] = sp[: min(n, sp.size)]
    want_f = orc.bf16_round(np.where(np.isnan(x), 0, x).astype(np.float32)).view(np.uint32) >> 16
    for doff in range(0, 16, 2):
        for soff in (0, 4):
            buf = np.full(2 * n + 64, 0xAB, np.uint8)
            src = np.zeros(n + 8, np.float32)
            src.view(np.uint8)[soff:soff + 4 * n] = x[:n].view(np.uint8)
            hc.hc_f2b(buf.ctypes.data + doff, src.ctypes.data + soff, n)
            got = buf[doff:doff + 2 * n].view(np.uint16)
            nan = np.isnan(x[:n])
            np.testing.assert_array_equal(got[~nan], want_f[:n][~nan].astype(np.uint16))
            xb = x[:n].view(np.uint32)
            assert np.all((got[nan] & 0x7FC0) == 0x7FC0)
            assert np.array_equal(got[nan] >> 15, (xb[nan] >> 31).astype(np.uint16))
            assert (buf[:doff] == 0xAB).all() and (buf[doff + 2 * n:] == 0xAB).all()


@pytest.mark.parametrize("n", LENGTHS)
def test_bf16_to_f32_every_alignment(hc, n):
    bits = np.random.default_rng(200 + n).integers(0, 1 << 16, n + 8, dtype=np.uint16)
    want = (bits[:n].astype(np.uint32) << 16)
    for doff in (0, 1, 2, 4, 8, 12):
        for soff in (0, 2, 6):
            src = np.zeros(2 * n + 16, np.uint8)
            src[soff:soff + 2 * n] = bits[:n].view(np.uint8)
            buf = np.full(4 * n + 64, 0xCD, np.uint8)
            hc.hc_b2f(buf.ctypes.data + doff, src.ctypes.data + soff, n)
            got = buf[doff:doff + 4 * n].copy().view(np.uint32)
            np.testing.assert_array_equal(got, want)
            assert (buf[:doff] == 0xCD).all() and (buf[doff + 4 * n:] == 0xCD).all()
