"""GPU parity of the single-matrix GEMV entries of the inner API, through the C-ABI:
affx_expert_gemv (expert_gemv_hip's arguments, src/gpu/expert_kernel_hip.h:147-148) and
affx_expert_gemv_batch (expert_gemv_batch_hip's, 152-153), the calls aff-gpucheck makes for its
per-matrix check and its GEMV bandwidth figure (tools/aff_gpucheck.cpp:278, 544-548). Each
matrix is uploaded on its own as aff-gpucheck does (host permutation, separate buffers) and the
result is compared with the oracle's expert_gemv_reference (y += w * W x, double accumulation)
at aff-gpucheck's own 1e-4 relative-L2 bar, at the benchmark shapes 2048 x 4096 (gate/up) and
4096 x 2048 (down)."""
import ctypes as C

import numpy as np
import pytest

from gpu_util import planes, random_expert_container, rel_l2

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

# aff-gpucheck fails a matrix whose GEMV differs from the CPU path by more than 1e-4 relative L2
# (tools/aff_gpucheck.cpp:295): the GEMVs are held to that bar, not to the FFN's 1e-3
TOL = 1e-4
H, I = 4096, 2048


@pytest.fixture(scope="module")
def ax():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import affinity_amd.experts as ax
    ax.init()
    return ax


def _upload(lib, ex, lay, which, rows, cols, keep):
    from affinity_amd._lib import AffxMatrix
    c, f, r = planes(ex, lay, which)
    dc, df = np.zeros_like(c), np.zeros_like(f)
    assert lib().affx_matrix_to_device_layout(c.ctypes.data, f.ctypes.data, dc.ctypes.data, df.ctypes.data,
                                              rows, cols) == 0
    bufs = [torch.from_numpy(a.view(np.uint8).copy()).cuda() for a in (dc, df, r)]
    keep.extend(bufs)
    return AffxMatrix(bufs[0].data_ptr(), bufs[1].data_ptr(), bufs[2].data_ptr(), rows, cols)


def _oracle(orc, ex, lay, which, rows, cols, cbf, x, w, y):
    c, f, r = planes(ex, lay, which)
    return orc.gemv(c, f, r, rows, cols, cbf, x, w, y)


@pytest.mark.parametrize("which,rows,cols", [(0, I, H), (2, H, I)])
def test_expert_gemv_single_matrix(ax, orc, c1_codebook, which, rows, cols):
    """y += w * W x for one matrix with a host weight; returns with y ready (no sync needed)."""
    from affinity_amd._lib import lib, last_error
    rng = np.random.default_rng(300 + which)
    lay = ax.expert_layout(H, I)
    ex = random_expert_container(rng, H, I, lay)
    keep = []
    m = _upload(lib, ex, lay, which, rows, cols, keep)
    cb = torch.from_numpy(c1_codebook.view(np.int32)).cuda()
    x = rng.standard_normal(cols).astype(np.float32)
    y0 = (0.1 * rng.standard_normal(rows)).astype(np.float32)
    xd, yd = torch.from_numpy(x).cuda(), torch.from_numpy(y0).cuda()
    assert lib().affx_expert_gemv(C.byref(m), cb.data_ptr(), xd.data_ptr(), 0.8, yd.data_ptr(), None) == 0, last_error()
    got = yd.cpu().numpy()
    ref = _oracle(orc, ex, lay, which, rows, cols, orc.unpack_codebook(c1_codebook), x, 0.8, y0.copy())
    err = rel_l2(got - y0, ref - y0)
    print(f"expert_gemv {rows}x{cols}: rel_l2 of the added term {err:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("which,rows,cols,n", [(0, I, H, 6), (2, H, I, 6), (1, I, H, 40)])
def test_expert_gemv_batch(ax, orc, c1_codebook, which, rows, cols, n):
    """y += sum_i w[i] W_i x over n matrices (40: two launches of at most 32), device weights."""
    from affinity_amd._lib import AffxMatrix, lib, last_error
    rng = np.random.default_rng(400 + n + which)
    lay = ax.expert_layout(H, I)
    cbf = orc.unpack_codebook(c1_codebook)
    keep = []
    mats = (AffxMatrix * n)()
    x = rng.standard_normal(cols).astype(np.float32)
    w = (0.05 + 0.9 * rng.random(n)).astype(np.float32)
    y0 = (0.1 * rng.standard_normal(rows)).astype(np.float32)
    ref = y0.copy()
    exs = [random_expert_container(rng, H, I, lay) for _ in range(min(n, 8))]
    for i in range(n):
        ex = exs[i % len(exs)]
        mats[i] = _upload(lib, ex, lay, which, rows, cols, keep)
        ref = _oracle(orc, ex, lay, which, rows, cols, cbf, x, float(w[i]), ref)
    cb = torch.from_numpy(c1_codebook.view(np.int32)).cuda()
    xd, yd, wd = (torch.from_numpy(a).cuda() for a in (x, y0, w))
    s = torch.cuda.current_stream().cuda_stream
    assert lib().affx_expert_gemv_batch(mats, wd.data_ptr(), n, cb.data_ptr(), xd.data_ptr(), yd.data_ptr(), s) == 0, \
        last_error()
    torch.cuda.synchronize()
    got = yd.cpu().numpy()
    err = rel_l2(got - y0, ref - y0)
    print(f"expert_gemv_batch {n} x {rows}x{cols}: rel_l2 of the added sum {err:.3e}")
    assert err <= TOL
    # the same call again on the same inputs: bit for bit (fixed summation order)
    yd2 = torch.from_numpy(y0).cuda()
    assert lib().affx_expert_gemv_batch(mats, wd.data_ptr(), n, cb.data_ptr(), xd.data_ptr(), yd2.data_ptr(), s) == 0
    torch.cuda.synchronize()
    assert torch.equal(yd2, yd)


def test_expert_gemv_declines_bad_shapes(ax, c1_codebook):
    from affinity_amd._lib import AFFX_DECLINED, AFFX_ERR_ARG, AffxMatrix, lib
    cb = torch.from_numpy(c1_codebook.view(np.int32)).cuda()
    buf = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    x = torch.zeros(8192 + 4, device="cuda")
    y = torch.zeros(4096, device="cuda")
    p = buf.data_ptr()
    for rows, cols in ((2048, 512), (2048, 1536), (2040, 1024), (16, 9216)):
        m = AffxMatrix(p, p, p, rows, cols)
        assert lib().affx_expert_gemv(C.byref(m), cb.data_ptr(), x.data_ptr(), 1.0, y.data_ptr(), None) == AFFX_DECLINED
    m = AffxMatrix(p, p, p, 16, 1024)
    assert lib().affx_expert_gemv(C.byref(m), cb.data_ptr(), x.data_ptr() + 4, 1.0, y.data_ptr(), None) == AFFX_ERR_ARG
    two = (AffxMatrix * 2)(AffxMatrix(p, p, p, 16, 1024), AffxMatrix(p, p, p, 32, 1024))
    assert lib().affx_expert_gemv_batch(two, y.data_ptr(), 2, cb.data_ptr(), x.data_ptr(), y.data_ptr(), None) == \
        AFFX_ERR_ARG
