"""The .aff container reader (affx_container_*), against a container the reference's own
AffWriter wrote and against the reference's own reader's addressing; and its refusals. The
GPU part uploads a layer and dequantises it bit for bit (test_gpu_container in this file)."""
import ctypes as C
import os
import shutil
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))


@pytest.fixture(scope="module")
def L():
    from affinity_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from affinity_amd.build import build
        build()
    return _lib.lib()


@pytest.fixture(scope="module")
def container(tmp_path_factory):
    from oracle import ref_available
    if not ref_available():
        pytest.skip("the reference build (its AffWriter) is not here")
    from make_container import write_small_container
    path = str(tmp_path_factory.mktemp("aff") / "small.aff")
    ex, cb = write_small_container(path)
    return path, ex, cb


def _open(L, path):
    h = C.c_void_p()
    rc = L.affx_container_open(path.encode(), C.byref(h))
    return rc, h


def test_reader_sees_what_the_reference_wrote(L, container):
    from oracle import load_ref
    path, ex, cb = container
    rc, h = _open(L, path)
    assert rc == 0, L.affx_last_error()
    try:
        assert L.affx_container_layer_count(h) == ex.shape[0]
        n, hid, inter, stride = C.c_uint32(), C.c_uint64(), C.c_uint64(), C.c_uint64()
        for l in range(ex.shape[0]):
            assert L.affx_container_layer(h, l, C.byref(n), C.byref(hid), C.byref(inter), C.byref(stride)) == 0
            assert (n.value, hid.value, inter.value) == (ex.shape[1], 1024, 1024)
            assert stride.value >= ex.shape[2]
        got = np.zeros(2048, np.uint32)
        assert L.affx_container_codebook(h, got.ctypes.data) == 0
        np.testing.assert_array_equal(got, cb)
        # every expert's bytes where the reference's reader puts them, and as written
        base = L.affx_container_expert_ptr(h, 0, 0)
        ref_off0 = load_ref().expert_offset(path, 0, 0)
        raw = np.fromfile(path, np.uint8)
        for l in range(ex.shape[0]):
            for e in range(ex.shape[1]):
                p = L.affx_container_expert_ptr(h, l, e)
                assert p - base == load_ref().expert_offset(path, l, e) - ref_off0
                mine = np.ctypeslib.as_array((C.c_uint8 * ex.shape[2]).from_address(p))
                np.testing.assert_array_equal(mine, ex[l, e])
                off = load_ref().expert_offset(path, l, e)
                np.testing.assert_array_equal(raw[off:off + ex.shape[2]], ex[l, e])
        assert not L.affx_container_expert_ptr(h, 0, ex.shape[1])
        assert not L.affx_container_expert_ptr(h, ex.shape[0], 0)
    finally:
        L.affx_container_close(h)


def test_reader_refuses_bad_files(L, container, tmp_path):
    path, _, _ = container
    raw = np.fromfile(path, np.uint8)

    def refused(data, why):
        p = str(tmp_path / "bad.aff")
        data.tofile(p)
        rc, h = _open(L, p)
        assert rc != 0, why
        assert why in L.affx_last_error().decode(), (why, L.affx_last_error())

    bad = raw.copy()
    bad[0] = ord("X")
    refused(bad, "bad magic")
    refused(raw[:-4096], "truncated")
    bad = raw.copy()
    bad[8] = 2                                                  # version
    refused(bad, "version")
    # the codebook: find the packed dwords and give one byte an exponent of 0
    cb = np.fromfile(os.path.join(HERE, "golden", "c1_codebook.bin"), np.uint8)
    at = raw.tobytes().find(cb.tobytes())
    assert at > 0
    bad = raw.copy()
    bad[at] = bad[at] & 0x87
    refused(bad, "exponent")
    # a layer whose gate matrix is declared in another format
    hdr = raw[:192].view(np.uint64)
    layer_dir = int(hdr[8])                                     # layer_dir_off
    bad = raw.copy()
    bad[layer_dir + 24 + 16] = 32                               # gate.quant = AFF_Q2P875
    refused(bad, "quad-format")
    # a layer stride whose product with the expert count wraps past 2^64 to a small extent
    n_exp = int(raw[layer_dir + 4:layer_dir + 8].view(np.uint32)[0])
    assert n_exp >= 2
    wrap = -(-(1 << 64) // n_exp)                               # n_exp * wrap = 2^64 + (< n_exp)
    bad = raw.copy()
    bad[layer_dir + 16:layer_dir + 24] = np.array([wrap], np.uint64).view(np.uint8)
    refused(bad, "corrupt layer descriptor")
    rc, h = _open(L, str(tmp_path / "missing.aff"))
    assert rc != 0


@pytest.mark.gpu
def test_gpu_container_upload_and_dequant(L, container, orc, c1_codebook):
    """affx_container_upload_layer puts each layer on the device byte for byte as the device-layout
    permutation of its container bytes, and dequantises to the oracle's floats bit for bit."""
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import affinity_amd.experts as ax
    from gpu_util import planes
    ax.init()
    path, ex, cb = container
    rc, h = _open(L, path)
    assert rc == 0, L.affx_last_error()
    try:
        stride, _, _ = ax.expert_layout(1024, 1024)
        n = ex.shape[1]
        staging = torch.empty(n * stride, dtype=torch.uint8, device="cuda")
        for l in range(ex.shape[0]):
            pool = ax.ExpertPool.empty(n, cb, 1024, 1024)
            assert L.affx_container_upload_layer(h, l, staging.data_ptr(), pool.data.data_ptr(),
                                                 torch.cuda.current_stream().cuda_stream) == 0
            ref = ax.ExpertPool.from_container(torch.from_numpy(ex[l].reshape(-1)).cuda(), cb, 1024, 1024)
            torch.cuda.synchronize()
            _, off, size = ax.expert_layout(1024, 1024)
            got, want = pool.data.view(n, stride), ref.data.view(n, stride)
            for p in range(9):
                assert torch.equal(got[:, off[p]:off[p] + size[p]], want[:, off[p]:off[p] + size[p]]), (l, p)
            cbf = orc.unpack_codebook(cb)
            lay = ax.expert_layout(1024, 1024)
            for e in range(n):
                for m in range(3):
                    d = ax.dequant_matrix(pool, e, m).cpu().numpy()
                    r = orc.dequantize(*planes(ex[l, e], lay, m), 1024, 1024, cbf)
                    np.testing.assert_array_equal(d.view(np.uint32), r.view(np.uint32))
    finally:
        L.affx_container_close(h)
