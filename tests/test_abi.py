"""CPU checks of the C-ABI library: it loads, exports every symbol include/affx.h declares, and
its host-side functions (geometry, codebook validation, the layout permutation) are right.
No GPU call is made here."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from gpu_util import random_expert_container

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "affx.h")


@pytest.fixture(scope="module")
def L():
    from affinity_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from affinity_amd.build import build
        build()
    return _lib.lib()


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(affx_[a-z0-9_]+)\s*\(", text)))


def test_exports_every_declared_symbol(L):
    names = header_functions()
    assert len(names) >= 15
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, f"libaffx.so lacks {missing}"


def test_python_binding_covers_header():
    from affinity_amd._lib import HEADER_SYMBOLS
    assert sorted(HEADER_SYMBOLS) == header_functions()


def layout(L, hidden, inter):
    off = (C.c_uint64 * 9)()
    size = (C.c_uint64 * 9)()
    stride = L.affx_expert_layout(hidden, inter, off, size)
    return int(stride), list(off), list(size)


def test_expert_layout_matches_container_geometry(L, orc):
    """Closed form at the V4 shapes (src/format/aff_format.cpp:45-91) and the oracle elsewhere."""
    stride, off, size = layout(L, 4096, 2048)
    assert stride == 9_060_352 == 2212 * 4096
    assert off == [0, 7_864_320, 9_043_968, 2_621_440, 8_257_536, 9_048_064, 5_242_880, 8_650_752, 9_052_160]
    assert size == [2_621_440, 393_216, 4096, 2_621_440, 393_216, 4096, 2_621_440, 393_216, 8192]
    for h, i in ((1024, 1024), (2048, 1024), (7168, 2048)):
        s, o, z = orc.expert_layout(h, i)
        assert layout(L, h, i) == (s, list(o), list(z))
    # 2.875 bits per weight plus the bf16 row scales
    n = 3 * 4096 * 2048
    assert sum(size) == n * 2.875 / 8 + 2 * (2048 * 2 + 4096)


def test_codebook_validation(L, c1_codebook):
    cb = np.ascontiguousarray(c1_codebook, np.uint32)
    assert L.affx_codebook_valid(cb.ctypes.data) == 1
    for bad_byte in (0x00, 0x40, 0xFF, 0x78):  # stored exponents 0, 8, 15, 15
        b = cb.copy()
        b.view(np.uint8)[1234] = bad_byte
        assert L.affx_codebook_valid(b.ctypes.data) == 0


def _numpy_to_device(src, hidden, inter, lay):
    """Independent statement of the device layout: unit (row r, 256-col segment u) -> tile
    (r//16)*(cols//1024) + u//4, lane r%16 + 16*(u%4); codes as five 1 KiB chunk planes, fields
    as 12 B per lane."""
    stride, off, size = lay
    dst = src.copy()
    for m, (rows, cols) in enumerate(((inter, hidden), (inter, hidden), (hidden, inter))):
        crow, frow, nst = cols * 10 // 32, cols * 6 // 128, cols // 1024
        c = src[off[3 * m]:off[3 * m] + size[3 * m]].reshape(rows, cols // 256, 5, 16)
        f = src[off[3 * m + 1]:off[3 * m + 1] + size[3 * m + 1]].reshape(rows, cols // 256, 12)
        c = c.reshape(rows // 16, 16, nst, 4, 5, 16).transpose(0, 2, 4, 3, 1, 5)  # rt st j g r b
        f = f.reshape(rows // 16, 16, nst, 4, 12).transpose(0, 2, 3, 1, 4)        # rt st g r b
        dst[off[3 * m]:off[3 * m] + size[3 * m]] = c.reshape(-1)
        dst[off[3 * m + 1]:off[3 * m + 1] + size[3 * m + 1]] = f.reshape(-1)
        assert crow * rows == size[3 * m] and frow * rows == size[3 * m + 1]
    return dst


@pytest.mark.parametrize("hidden,inter", [(1024, 1024), (4096, 2048)])
def test_host_permutation_is_the_stated_bijection(L, hidden, inter):
    rng = np.random.default_rng(3)
    lay = layout(L, hidden, inter)
    src = random_expert_container(rng, hidden, inter, lay)
    dev = np.zeros_like(src)
    back = np.zeros_like(src)
    assert L.affx_expert_to_device_layout(src.ctypes.data, dev.ctypes.data, hidden, inter) == 0
    np.testing.assert_array_equal(dev, _numpy_to_device(src, hidden, inter, lay))
    assert L.affx_expert_from_device_layout(dev.ctypes.data, back.ctypes.data, hidden, inter) == 0
    np.testing.assert_array_equal(back, src)


@pytest.mark.parametrize("hidden,inter", [(1024, 1024), (4096, 2048)])
def test_matrix_permutation_composes_to_the_expert_permutation(L, hidden, inter):
    """affx_matrix_to_device_layout on each matrix's own planes (separate buffers, as aff-gpucheck
    uploads them) gives the same bytes as the whole-expert permutation at those planes."""
    rng = np.random.default_rng(4)
    lay = layout(L, hidden, inter)
    _, off, size = lay
    src = random_expert_container(rng, hidden, inter, lay)
    dev = np.zeros_like(src)
    assert L.affx_expert_to_device_layout(src.ctypes.data, dev.ctypes.data, hidden, inter) == 0
    for m, (rows, cols) in enumerate(((inter, hidden), (inter, hidden), (hidden, inter))):
        c = np.ascontiguousarray(src[off[3 * m]:off[3 * m] + size[3 * m]])
        f = np.ascontiguousarray(src[off[3 * m + 1]:off[3 * m + 1] + size[3 * m + 1]])
        dc, df = np.zeros_like(c), np.zeros_like(f)
        assert L.affx_matrix_to_device_layout(c.ctypes.data, f.ctypes.data, dc.ctypes.data, df.ctypes.data,
                                              rows, cols) == 0
        np.testing.assert_array_equal(dc, dev[off[3 * m]:off[3 * m] + size[3 * m]])
        np.testing.assert_array_equal(df, dev[off[3 * m + 1]:off[3 * m + 1] + size[3 * m + 1]])
    assert L.affx_matrix_to_device_layout(c.ctypes.data, f.ctypes.data, dc.ctypes.data, df.ctypes.data, 15, 1024) < 0


def test_bad_arguments_are_refused(L):
    buf = np.zeros(16, np.uint8)
    assert L.affx_expert_to_device_layout(buf.ctypes.data, buf.ctypes.data, 4096, 2048) < 0
    assert L.affx_expert_to_device_layout(buf.ctypes.data, None, 4096, 2048) < 0
    assert b"bad arguments" in L.affx_last_error()


def test_grouped_refuses_misaligned_activations(L):
    """The grouped prefill reads x with 16-byte loads: a misaligned x or x_lo is an argument error,
    refused before any device work (so this runs without a GPU)."""
    from affinity_amd._lib import AffxLayer
    buf = np.zeros(64, np.uint8)
    p = buf.ctypes.data
    lay = AffxLayer(p, 9060352, 256, 4096, 2048, p, 10.0)
    for x, xlo in ((p + 2, None), (p, p + 8)):
        rc = L.affx_expert_ffn_grouped(C.byref(lay), x, xlo, 4, p, p, 6, p, 0, p, 1 << 30, None)
        assert rc == -1, rc  # AFFX_ERR_ARG
        assert b"16-byte aligned" in L.affx_last_error()


def test_decode_workspace_grows_with_batch(L):
    a = L.affx_decode_workspace_size(1, 6, 4096, 2048)
    b = L.affx_decode_workspace_size(8, 6, 4096, 2048)
    assert 0 < a < b
